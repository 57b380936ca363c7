"""CPU check of the argument behind the Q8_1 quantiser's division shortcut
(csrc/q8_1_block.h, round_codes): with r = 1/d from a reciprocal instruction
that is within 1 ulp, p = x*r rounds to the same integer as roundf(x/d)
whenever |frac(|p|) - 1/2| >= 2^-14; a lane holding any other value
recomputes its values by the exact division (which is right for all of
them).  Emulated here in numpy with r perturbed by -1, 0 and +1 ulp and
compared with the oracle's codes, on blocks built to sit on and near the
rounding boundaries and on ordinary activations."""
import numpy as np

from oracle.oracle import Q8_1_BYTES

THRESH = np.float32(2.0**-14)


def boundary_blocks(n_blocks: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    offs = np.array([0.0, 2.0**-24, -2.0**-24, 2.0**-18, -2.0**-18, 2.0**-15, -2.0**-15,
                     2.0**-14, -2.0**-14, 2.0**-12, -2.0**-12])
    out = np.zeros((n_blocks, 32), np.float32)
    for b in range(n_blocks):
        amax = np.float32(10.0 ** rng.uniform(-30, 30))
        d = np.float32(amax / np.float32(127.0))
        k = rng.integers(-127, 127, 32)
        out[b] = ((k + 0.5 + rng.choice(offs, 32)) * np.float64(d)).astype(np.float32)
        out[b, rng.integers(32)] = amax * rng.choice([-1.0, 1.0])
    return out


def fast_codes(xb: np.ndarray, ulp_shift: int):
    """(codes, taken) of the shortcut; taken = lanes that skip the division."""
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        r = (np.float32(1.0) / d).astype(np.float32)
        if ulp_shift:
            r = np.nextafter(r, np.float32(np.inf) if ulp_shift > 0 else np.float32(0.0)).astype(np.float32)
        p = (xb * r[:, None]).astype(np.float32)
        ap = np.abs(p)
        f = (ap - np.floor(ap)).astype(np.float32)
        taken = np.abs((f - np.float32(0.5)).astype(np.float32)) >= THRESH
        q = np.trunc((p + np.copysign(np.float32(0.5), p)).astype(np.float32))
    return q, taken


def test_shortcut_agrees_with_exact_division(orc):
    rng = np.random.default_rng(3)
    xb = np.concatenate([boundary_blocks(4096, seed=4),
                         rng.standard_normal((4096, 32)).astype(np.float32),
                         (rng.standard_normal((1024, 32)) * 1e-3).astype(np.float32)])
    ref = orc.quantize_q8_1(xb.ravel()).reshape(-1, Q8_1_BYTES)
    q_ref = ref[:, 4:].view(np.int8).astype(np.float32)
    n_slow = 0
    for shift in (-1, 0, 1):
        q, taken = fast_codes(xb, shift)
        assert np.array_equal(q[taken], q_ref[taken]), shift
        n_slow += int((~taken).sum())
    # the boundary blocks really do reach the exact path, and the shortcut
    # would have been wrong on some of those lanes
    q0, taken0 = fast_codes(xb, 0)
    assert n_slow > 1000
    assert np.any(q0[~taken0] != q_ref[~taken0])
