"""ozk_matmul_noalloc against ozk_matmul, through the C ABI.

The no-allocation entry point runs ozk_matmul on the library's own scratch
array; its results must be bit-identical to ozk_matmul's with a caller
workspace (np.array_equal, NaN == NaN), on two calls in a row, the second
with a smaller input (the array keeps the first call's contents), for the
INT8- and BF16-plane on-device paths and the host pipeline.  Shapes whose
workspace exceeds the array are refused before any device work.
"""

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _run(lib, A, B, pipeline, nh, nl, order, noalloc):
    import torch
    from ozaki_jax_amd import _device as D, _lib
    dev = torch.device("cuda", 0)
    At = torch.from_numpy(A).to(dev)
    Bt = torch.from_numpy(B).to(dev)
    N, K = A.shape
    M = B.shape[1]
    C = torch.full((N, M), 7.0, dtype=torch.float64, device=dev)
    flags = torch.full((1,), -1, dtype=torch.int32, device=dev)
    if noalloc:
        rc = lib.ozk_matmul_noalloc(At.data_ptr(), K, Bt.data_ptr(), M, C.data_ptr(), M,
                                    N, K, M, pipeline, nh, nl, order, flags.data_ptr(),
                                    D.stream_handle())
    else:
        wsb = lib.ozk_matmul_workspace_bytes(N, K, M, pipeline, nh, nl)
        ws = D.workspace(wsb, dev)
        rc = lib.ozk_matmul(At.data_ptr(), K, Bt.data_ptr(), M, C.data_ptr(), M, N, K, M,
                            pipeline, nh, nl, order, ws.data_ptr(), wsb, flags.data_ptr(),
                            D.stream_handle())
    _lib.check(rc)
    return C.cpu().numpy(), int(flags.item())


# (first call, second smaller call) per path
SEQUENCES = [
    ("INT8 planes, high, 2Sum", 0, 4, 1, 0, (600, 5000, 576), (130, 4200, 90)),
    ("INT8 planes, max, block order", 0, 5, 4, 1, (300, 6000, 280), (70, 4500, 33)),
    ("BF16 planes, high, 2Sum", 0, 4, 1, 0, (1100, 2048, 1000), (96, 300, 64)),
    ("host pipeline, n_slices=8", 1, 8, 0, 3, (256, 256, 256), (40, 100, 30)),
    ("INT8 planes, (6, 1) rectangle sweeps, 2Sum", 0, 6, 1, 0, (600, 5000, 576), (130, 4200, 90)),
]


@pytest.mark.parametrize("name,pipe,nh,nl,order,first,second", SEQUENCES)
def test_noalloc_matches_workspace_entry(ozk, name, pipe, nh, nl, order, first, second):
    from ozaki_jax_amd import _lib
    lib = _lib.load()
    rng = np.random.RandomState(len(name))
    for N, K, M in (first, second):
        assert lib.ozk_matmul_workspace_bytes(N, K, M, pipe, nh, nl) <= 128 << 20
        A = rng.randn(N, K)
        B = (rng.rand(K, M) - 0.5) * np.exp(2.0 * rng.randn(K, M))
        if N > 64:
            A[3] *= 2.0 ** -110   # a NaN row on INT8 planes, as with ozk_matmul
        case(f"ozk_matmul_noalloc {name} ({N},{K},{M})")
        Cn, fn = _run(lib, A, B, pipe, nh, nl, order, True)
        Cw, fw = _run(lib, A, B, pipe, nh, nl, order, False)
        assert np.array_equal(Cn, Cw, equal_nan=True)
        assert fn == fw
        assert np.isfinite(Cn).sum() >= (N - 1) * M


def test_noalloc_refuses_shapes_above_the_scratch(ozk):
    from ozaki_jax_amd import _lib
    lib = _lib.load()
    cap = 128 << 20
    assert lib.ozk_matmul_workspace_bytes(4096, 4096, 4096, 0, 4, 1) > cap
    assert lib.ozk_matmul_workspace_bytes(2048, 2048, 2048, 0, 4, 1) <= cap
    case("ozk_matmul_noalloc 4096^3 high: refused")
    rc = lib.ozk_matmul_noalloc(None, 4096, None, 4096, None, 4096, 4096, 4096, 4096, 0, 4,
                                1, 0, None, None)
    assert rc == _lib.OZK_ERR_WORKSPACE
    assert b"scratch" in lib.ozk_last_error()
    case("ozk_matmul_noalloc bad slice count: refused")
    assert lib.ozk_matmul_noalloc(None, 8, None, 8, None, 8, 8, 8, 8, 0, 0, 1, 0, None,
                                  None) == _lib.OZK_ERR_INVALID
