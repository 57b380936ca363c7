"""The kernels on matmul fixtures in the reference's format
(tests/golden/matmul_fixtures, cut from a synthetic GGUF by this package's
reader): weights uploaded from the GGUF file itself, activations and y_ref
from the fixture files.  Gates: the reference's own for its real-weight
comparison (cosine >= 0.99 and no NaN/Inf against y_ref,
kernels/matmul_iq4xs/test_real_stock_compare.cpp:40-41), and the path's
bar of rel-L2 <= 1e-4 against the oracle's kernel semantics."""
import ctypes
import importlib
import os

import numpy as np
import pytest

from oracle.oracle import LAYOUT_KM, compute_metrics

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

FIXDIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "matmul_fixtures")


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


def test_fixture_cases_through_reference_entry_points(pkg, orc, dev):
    gg = importlib.import_module(pkg.__name__ + ".gguf")
    fx = importlib.import_module(pkg.__name__ + ".fixtures")
    L = pkg.lib()
    s = torch.cuda.current_stream().cuda_stream
    entries = fx.load_manifest(FIXDIR)
    assert entries
    with gg.GGUFReader(os.path.join(FIXDIR, "synthetic_layer.gguf")) as r:
        for e in entries:
            c = fx.load_matmul_case(FIXDIR, e)
            K, N, M = c["K"], c["N"], c["M"]
            print(f"fixture {e['name']} K={K} N={N} M={M}", flush=True)
            W_np = fx.extract_projection(r, e["W_source"], K, N)
            assert np.array_equal(W_np, c["W"])          # the GGUF holds what the fixture says
            W = gg.to_device(W_np, dev)
            X = torch.from_numpy(np.ascontiguousarray(c["X"])).to(dev)     # [K][M]: X[k*M + m]
            Y = torch.empty((N, M), device=dev)                             # Y[n*M + m]
            if M == 1:
                L.check("gemv_iq4xs_stock_dp4a_gpu", W.data_ptr(), X.data_ptr(), Y.data_ptr(), K, N, s)
            else:
                L.check("gemm_iq4xs_stock_dp4a_gpu", W.data_ptr(), X.data_ptr(), Y.data_ptr(), K, N, M, s)
            got = Y.cpu().numpy()
            ref_gate = compute_metrics(c["Y_ref"], got)
            assert not ref_gate["bad"] and ref_gate["cosine"] >= 0.99, (e["name"], M, ref_gate)
            AQ = orc.quantize_q8_1_batched(c["X"], K, M, LAYOUT_KM)
            sem = compute_metrics(orc.gemm_semantics(c["W"], AQ, K, N, M), got)
            assert sem["rel_l2"] <= 1e-4 and not sem["bad"], (e["name"], M, sem)
