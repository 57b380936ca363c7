"""Graph capture: the entry points a decode or prefill step calls, captured
into one HIP graph on a side stream and replayed several times, with eager
work and synchronisation between the replays.  Every replay must give the
eager run's outputs bit for bit (the outputs are overwritten with NaN before
each replay, so a node that did not run would show).  Covered: the fused
single-column GEMV (two- and five-round prologues), the quantiser + GEMM,
the quantiser + matrix-core small-batch GEMV, grouped GEMVs (tile and
matrix-core), the rms-fused grouped GEMV, the rms + gate/up + SwiGLU launch
and the down GEMV on its output, the allocation-free entry point and the
ggml GEMV hook.  None of
them records a memset or an allocation into the graph."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


def bits(t):
    return t.contiguous().cpu().numpy().view(np.uint32)


def test_graph_replays_match_eager(pkg, dev):
    L = pkg.lib()
    side = torch.cuda.Stream()
    H, Q, FF = 5120, 8192, 17408
    g = torch.Generator().manual_seed(77)
    with torch.cuda.stream(side):
        s = side.cuda_stream
        Wq = pkg.synthetic_weights(H, Q, seed=1, device=dev)
        Wk = pkg.synthetic_weights(H, 1024, seed=2, device=dev)
        Wg = pkg.synthetic_weights(H, FF, seed=3, device=dev)
        Wu = pkg.synthetic_weights(H, FF, seed=4, device=dev)
        Wd = pkg.synthetic_weights(FF, H, seed=5, device=dev)
        x = (torch.randn(H, generator=g) * 2.0).to(dev)
        r = (torch.randn(H, generator=g) * 0.5).to(dev)
        gamma = (torch.rand(H, generator=g) + 0.5).to(dev)
        xff = torch.randn(FF, generator=g).to(dev)
        X4 = torch.randn((4, H), generator=g).to(dev)
        X8 = torch.randn((8, H), generator=g).to(dev)
        X64 = torch.randn((64, H), generator=g).to(dev)
        ws = {k: pkg.workspace(K, M, dev) for k, (K, M) in
              {"q": (H, 1), "d": (FF, 1), "m4": (H, 4), "m8": (H, 8), "m64": (H, 64), "s": (FF, 1)}.items()}
        out = {"q": torch.empty(Q, device=dev), "d": torch.empty(H, device=dev),
               "m4": torch.empty((4, Q), device=dev), "m64": torch.empty((64, Q), device=dev),
               "gq": torch.empty(Q, device=dev), "gk": torch.empty(1024, device=dev),
               "rq": torch.empty(Q, device=dev), "rk": torch.empty(1024, device=dev),
               "h1": torch.empty(H, device=dev), "h2": torch.empty(H, device=dev),
               "S": torch.empty(FF, device=dev), "gate": torch.empty(FF, device=dev),
               "up": torch.empty(FF, device=dev), "down": torch.empty(H, device=dev),
               "noalloc": torch.empty(1024, device=dev), "hook": torch.empty(1024, device=dev),
               "g8q": torch.empty((8, Q), device=dev), "g8k": torch.empty((8, 1024), device=dev),
               "g8v": torch.empty((8, 1024), device=dev), "g4g": torch.empty((4, FF), device=dev),
               "g4u": torch.empty((4, FF), device=dev)}

        def step():
            pkg.mul_mat(Wq, x, H, Q, 1, ws=ws["q"], out=out["q"])             # fused, two rounds
            pkg.mul_mat(Wd, xff, FF, H, 1, ws=ws["d"], out=out["d"])          # fused, five rounds
            pkg.mul_mat(Wq, X4, H, Q, 4, ws=ws["m4"], out=out["m4"])          # quantiser + matrix-core GEMV
            pkg.mul_mat(Wq, X64, H, Q, 64, ws=ws["m64"], out=out["m64"])      # quantiser + GEMM
            pkg.mul_mat_q8_1_group([Wq, Wk], ws["q"], H, [Q, 1024], 1, outs=[out["gq"], out["gk"]])
            # matrix-core GEMV groups: q/k/v in one launch at 8 columns, gate/up in one at 4
            pkg.quantize_q8_1(X8, H, 8, ws=ws["m8"])
            pkg.mul_mat_q8_1_group([Wq, Wk, Wk], ws["m8"], H, [Q, 1024, 1024], 8,
                                   outs=[out["g8q"], out["g8k"], out["g8v"]])
            pkg.mul_mat_q8_1_group([Wg, Wu], ws["m4"], H, [FF, FF], 4, outs=[out["g4g"], out["g4u"]])
            pkg.rms_norm_mul_mat_group([Wq, Wk], x, H, [Q, 1024], residual=r, out_h=out["h1"], gamma=gamma,
                                       outs=[out["rq"], out["rk"]])
            pkg.rms_norm_mul_mat_swiglu(Wg, Wu, out["h1"], H, FF, residual=x, out_h=out["h2"], gamma=gamma,
                                        gate_out=out["gate"], up_out=out["up"], out=out["S"])
            pkg.mul_mat(Wd, out["S"], FF, H, 1, ws=ws["s"], out=out["down"])
            L.check("iq4xs_mul_mat_noalloc", Wk.data_ptr(), x.data_ptr(), out["noalloc"].data_ptr(), H, 1024, 1,
                    pkg.LAYOUT_MK, s)
            L.check("custom_gemv_iq4xs_dispatch", Wk.data_ptr(), x.data_ptr(), out["hook"].data_ptr(), H, 1024, s)

        step()
        side.synchronize()
        ref = {k: bits(v) for k, v in out.items()}
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            step()
        for rep in range(4):
            print(f"[graphs] replay {rep}", flush=True)
            for v in out.values():
                v.fill_(float("nan"))
            graph.replay()
            side.synchronize()
            for k, v in out.items():
                assert np.array_equal(bits(v), ref[k]), (rep, k)
            # eager work between replays, on other inputs
            pkg.mul_mat(Wq, X4 * 2.0, H, Q, 4)
            pkg.mul_mat(Wk, xff[:H] * 3.0, H, 1024, 1)
            side.synchronize()
