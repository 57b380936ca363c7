"""Whole-model weight stream (64 layers of the 27B-class decode projections,
12.30 GB of IQ4_XS resident): bench.py's own chain (bench.ModelChain) on the
GPU, checked against the oracle.

* Two layers through every variant -- plain, grouped, rms-fused and
  rms+swiglu-fused at bs=1, plain and grouped at M=512 -- at the full
  config-1 shapes: every producer's Q8_1 blocks (and the residual stream h)
  bit for bit against the oracle's rms norm / swiglu, the fused SwiGLU's fp32
  silu(gate) * up bit for bit against the oracle's; every projection on
  sampled rows within rel-L2 1e-4 of the reference GEMM semantics on the
  blocks it read.
* The full 64-layer bs=1 chain: finite, the four variants bit-identical to
  each other, and a replay bit-identical to the first run.
* The full 64-layer M=512 pass: finite, grouped bit-identical to plain.
"""
import numpy as np
import pytest

from oracle.oracle import LAYOUT_MK, compute_metrics

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-4
ROWS_PER_PROJ = 16


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def bench():
    import bench as b

    return b


@pytest.fixture(scope="module")
def model(pkg, bench, dev):
    stream = torch.cuda.current_stream()
    w = bench.make_model_weights(torch, pkg.lib(), 64, stream, dev)
    torch.cuda.synchronize()
    yield w
    del w
    torch.cuda.empty_cache()


def bits(t):
    return t.contiguous().cpu().numpy().view(np.uint32)


class Checker:
    """Stage callback of bench.ModelChain: each stage against the oracle."""

    def __init__(self, pkg, orc, bench, weights, M):
        self.pkg, self.orc, self.bench, self.weights, self.M = pkg, orc, bench, weights, M
        self.shapes = {name: (i, K, N) for i, (name, K, N) in enumerate(bench.SHAPES)}
        self.gain = np.full(bench.SHAPES[0][1], bench.MODEL_GAIN, np.float32)
        self.seen = []

    def blocks(self, ws, K):
        return self.pkg.q8_1_blocks(ws, K, self.M).cpu().numpy().ravel()

    def rms(self, l, stage, h_in, r_in, h_out):
        K = self.bench.SHAPES[0][1]
        H, _, Q = self.orc.rms_norm_q8_1(h_in.cpu().numpy(), K, self.M, R=r_in.cpu().numpy(), gamma=self.gain,
                                         eps=self.bench.MODEL_EPS)
        assert np.array_equal(bits(h_out), H.view(np.uint32).reshape(bits(h_out).shape)), (l, stage, "h")
        return Q

    def proj(self, l, stage, name, AQ, Y):
        i, K, N = self.shapes[name]
        rows = np.sort(np.random.default_rng(1000 * l + i).choice(N, ROWS_PER_PROJ, replace=False))
        W = self.weights[l][i].view(N, -1)[torch.from_numpy(rows).to(Y.device)].cpu().numpy().ravel()
        Y_sem = self.orc.gemm_semantics(W, AQ, K, len(rows), self.M).T
        m = compute_metrics(Y_sem, Y.cpu().numpy()[:, rows])
        assert m["rel_l2"] <= REL_L2_TOL and not m["bad"], (l, stage, name, m)
        assert bool(torch.isfinite(Y).all()), (l, stage, name)

    def __call__(self, l, stage, **t):
        print(f"[model-stream] M={self.M} layer {l} stage {stage}", flush=True)
        self.seen.append(stage)
        H_DIM, Q_DIM, FF_DIM = self.bench.SHAPES[0][1], self.bench.SHAPES[0][2], self.bench.SHAPES[4][2]
        if stage in ("rms_attn", "rms_ffn"):
            Q = self.rms(l, stage, t["h_in"], t["r_in"], t["h_out"])
            assert np.array_equal(self.blocks(t["ws"], H_DIM), Q), (l, stage, "Q8_1")
        elif stage in ("rms_qkv_fused", "rms_gate_up_fused"):
            Q = self.rms(l, stage, t["h_in"], t["r_in"], t["h_out"])
            names = ("q_proj", "k_proj", "v_proj") if stage == "rms_qkv_fused" else ("gate_proj", "up_proj")
            keys = ("q", "k", "v") if stage == "rms_qkv_fused" else ("gate", "up")
            for name, key in zip(names, keys):
                self.proj(l, stage, name, Q, t[key])
        elif stage == "qkv":
            AQ = self.blocks(t["ws"], H_DIM)
            for name, key in (("q_proj", "q"), ("k_proj", "k"), ("v_proj", "v")):
                self.proj(l, stage, name, AQ, t[key])
        elif stage == "gate_up":
            AQ = self.blocks(t["ws"], H_DIM)
            for name, key in (("gate_proj", "gate"), ("up_proj", "up")):
                self.proj(l, stage, name, AQ, t[key])
        elif stage == "o":
            AQ = self.orc.quantize_q8_1_batched(t["x"].cpu().numpy(), Q_DIM, self.M, LAYOUT_MK)
            self.proj(l, stage, "o_proj", AQ, t["o"])
        elif stage == "swiglu":
            _, Q = self.orc.swiglu_q8_1(t["gate"].cpu().numpy(), t["up"].cpu().numpy(), FF_DIM, self.M)
            assert np.array_equal(self.blocks(t["ws"], FF_DIM), Q), (l, "swiglu", "Q8_1")
        elif stage == "down":
            self.proj(l, stage, "down_proj", self.blocks(t["ws"], FF_DIM), t["down"])
        elif stage == "rms_gate_up_swiglu":
            Q = self.rms(l, stage, t["h_in"], t["r_in"], t["h_out"])
            for name, key in (("gate_proj", "gate"), ("up_proj", "up")):
                self.proj(l, stage, name, Q, t[key])
            g, u = t["gate"].cpu().numpy().ravel(), t["up"].cpu().numpy().ravel()
            S_ref = (self.orc.silu(g) * u).astype(np.float32)
            assert np.array_equal(bits(t["s"]).ravel(), S_ref.view(np.uint32)), (l, stage, "S")
        elif stage == "down_from_s":
            AQ = self.orc.quantize_q8_1_batched(t["x"].cpu().numpy(), FF_DIM, self.M, LAYOUT_MK)
            self.proj(l, stage, "down_proj", AQ, t["down"])
        else:
            raise AssertionError(stage)


@pytest.mark.parametrize("M,variant", [(1, "plain"), (1, "grouped"), (1, "fused"), (1, "fused_swiglu"),
                                       (512, "plain"), (512, "grouped")])
def test_two_layers_against_oracle(pkg, orc, bench, model, dev, M, variant):
    print(f"[model-stream] two checked layers M={M} variant={variant}", flush=True)
    chain = bench.ModelChain(torch, pkg, pkg.lib(), model, M, torch.cuda.current_stream(), variant)
    chk = Checker(pkg, orc, bench, model, M)
    chain.run(2, check=chk)
    assert chain.finite()
    per_layer = {"fused": 5, "fused_swiglu": 4}.get(variant, 7)
    assert len(chk.seen) == 2 * per_layer


def test_64_layers_bs1_variants_bit_identical(pkg, bench, model, dev):
    stream = torch.cuda.current_stream()
    states = {}
    for variant in ("plain", "grouped", "fused", "fused_swiglu", "plain"):
        print(f"[model-stream] 64 layers bs=1 variant={variant}", flush=True)
        chain = bench.ModelChain(torch, pkg, pkg.lib(), model, 1, stream, variant)
        chain.run()
        assert chain.finite(), variant
        snap = [bits(t) for t in chain.state()]
        if variant in states:  # the replay: a fresh chain from the same seed
            assert all(np.array_equal(a, b) for a, b in zip(states[variant], snap)), "replay differs"
        states[variant] = snap
        del chain
    for variant in ("grouped", "fused", "fused_swiglu"):
        for j, (a, b) in enumerate(zip(states["plain"], states[variant])):
            assert np.array_equal(a, b), (variant, j)
    # the chain did run: the last layer's outputs are not the initial zeros
    assert np.any(states["plain"][-1] != 0)


def test_64_layers_bs512_grouped_bit_identical(pkg, bench, model, dev):
    """The whole-model prefill pass (M = 512 through all 64 layers, producers and the q
    re-quantisation included): finite, and with the grouped launches (q/k/v and gate/up one
    iq4xs_mul_mat_q8_1_group each) bit-identical to one call per projection -- the residual
    stream h after layer 64 and the last layer's seven outputs, which every earlier layer
    feeds."""
    stream = torch.cuda.current_stream()
    states = {}
    for variant in ("plain", "grouped"):
        print(f"[model-stream] 64 layers M=512 variant={variant}", flush=True)
        chain = bench.ModelChain(torch, pkg, pkg.lib(), model, 512, stream, variant)
        chain.run()
        assert chain.finite(), variant
        states[variant] = [bits(t) for t in chain.state()]
        del chain
    for j, (a, b) in enumerate(zip(states["plain"], states["grouped"])):
        assert np.array_equal(a, b), j
    assert np.any(states["plain"][-1] != 0)
