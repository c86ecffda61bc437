"""ozk_matmul_early_flags against ozk_matmul through the C ABI.

The early-flag entry point runs ozk_matmul and also copies the call's flag
word to a pinned host word, with an event recorded after the copy, as soon as
the extraction (the only kernels that set flags) is queued.  The product and
the device flag word must equal ozk_matmul's bit for bit, and the host word
must equal the device word: on INT8 and BF16 planes, with NaN input
(OZK_FLAG_NONFINITE), with rows whose slices overflow (the INT8 planes'
OZK_FLAG_INF_SLICE), and for an empty product.
"""

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


CASES = [((130, 8192, 70), 4, 1, 0, None),
         ((130, 8192, 70), 4, 1, 0, "nan"),
         ((64, 8192, 48), 4, 1, 1, "big"),
         ((64, 8192, 48), 5, 4, 0, "tiny"),
         ((100, 300, 90), 3, 1, 0, None),
         ((100, 300, 90), 4, 1, 1, "nan"),
         ((0, 300, 90), 4, 1, 0, None)]


@pytest.mark.parametrize("shape,nh,nl,order,kind", CASES)
def test_early_flags_match_matmul(ozk, shape, nh, nl, order, kind):
    import torch
    from ozaki_jax_amd import _lib, _device as D
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    N, K, M = shape
    rng = np.random.RandomState(N + K + M + nh)
    A, B = rng.randn(N, K), rng.randn(K, M)
    if kind == "nan" and N:
        A[N // 2, K // 3] = np.nan
    elif kind == "big":
        A[1] *= 2.0 ** 110
    elif kind == "tiny":
        A[2] *= 2.0 ** -110
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    pipe = _lib.PIPE_ONDEVICE
    wsb = lib.ozk_matmul_workspace_bytes(N, K, M, pipe, nh, nl)
    ws = D.workspace(wsb, dev)

    def args(C, flags):
        return (At.data_ptr(), D.ld_of(At), Bt.data_ptr(), D.ld_of(Bt), C.data_ptr(),
                D.ld_of(C), N, K, M, pipe, nh, nl, order, ws.data_ptr(), wsb,
                flags.data_ptr())

    case(f"ozk_matmul vs ozk_matmul_early_flags {shape} ({nh},{nl}) order {order} {kind}")
    C1 = torch.full((N, M), 7.0, dtype=torch.float64, device=dev)
    f1 = torch.full((1,), -559038737, dtype=torch.int32, device=dev)
    _lib.check(lib.ozk_matmul(*args(C1, f1), D.stream_handle()))
    fl1 = int(f1.item()) & 0xffffffff

    word, ev, read = D._TorchFamily().early_flags()
    C2 = torch.full((N, M), 7.0, dtype=torch.float64, device=dev)
    f2 = torch.full((1,), -559038737, dtype=torch.int32, device=dev)
    _lib.check(lib.ozk_matmul_early_flags(*args(C2, f2), word, ev, D.stream_handle()))
    early = read()
    torch.cuda.synchronize()
    assert early == int(f2.item()) & 0xffffffff == fl1
    if kind == "nan":
        assert fl1 & _lib.OZK_FLAG_NONFINITE
    elif kind is None:
        assert fl1 == 0
    assert np.array_equal(C1.cpu().numpy(), C2.cpu().numpy(), equal_nan=True)


@pytest.mark.parametrize("rows,cols,nh,nl,kind", [(9000, 200, 4, 1, None), (9000, 200, 4, 1, "nan"),
                                                  (3000, 150, 5, 4, None), (300, 0, 4, 1, None)])
def test_gram_early_flags_match_gram(ozk, rows, cols, nh, nl, kind):
    import torch
    from ozaki_jax_amd import _lib, _device as D
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    rng = np.random.RandomState(rows + cols)
    A = rng.randn(rows, cols)
    if kind == "nan":
        A[rows // 2, cols // 3] = np.nan
    At = torch.from_numpy(A).to(dev)
    wsb = lib.ozk_gram_workspace_bytes(rows, cols, nh, nl)
    ws = D.workspace(wsb, dev)

    def run(fn, *extra):
        G = torch.full((cols, cols), 7.0, dtype=torch.float64, device=dev)
        f = torch.full((1,), -559038737, dtype=torch.int32, device=dev)
        _lib.check(fn(At.data_ptr(), D.ld_of(At), rows, cols, nh, nl, G.data_ptr(),
                      max(cols, 1), ws.data_ptr(), wsb, f.data_ptr(), *extra,
                      D.stream_handle()))
        return G, f

    case(f"ozk_gram vs ozk_gram_early_flags ({rows},{cols}) ({nh},{nl}) {kind}")
    G1, f1 = run(lib.ozk_gram)
    fl1 = int(f1.item()) & 0xffffffff
    word, ev, read = D._TorchFamily().early_flags()
    G2, f2 = run(lib.ozk_gram_early_flags, word, ev)
    early = read()
    torch.cuda.synchronize()
    assert early == int(f2.item()) & 0xffffffff == fl1
    assert (fl1 & _lib.OZK_FLAG_NONFINITE) == (kind == "nan")
    assert np.array_equal(G1.cpu().numpy(), G2.cpu().numpy(), equal_nan=True)


def test_early_flags_rejects_null_host_word(ozk):
    import torch
    from ozaki_jax_amd import _lib, _device as D
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    A = torch.ones((8, 8), dtype=torch.float64, device=dev)
    C = torch.empty((8, 8), dtype=torch.float64, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    case("ozk_matmul_early_flags / ozk_gram_early_flags with a null host word")
    with pytest.raises(ValueError, match="host flag word"):
        _lib.check(lib.ozk_matmul_early_flags(
            A.data_ptr(), 8, A.data_ptr(), 8, C.data_ptr(), 8, 8, 8, 8,
            _lib.PIPE_ONDEVICE, 4, 1, 0, None, 0, flags.data_ptr(), None, None,
            D.stream_handle()))
    with pytest.raises(ValueError, match="host flag word"):
        _lib.check(lib.ozk_gram_early_flags(
            A.data_ptr(), 8, 8, 8, 4, 1, C.data_ptr(), 8, None, 0, flags.data_ptr(),
            None, None, D.stream_handle()))


def test_torch_matmul_returns_before_the_product_and_raises_on_nan(ozk):
    """The torch family reads the flags early: results are still bit-exact,
    NaN input still raises, and safe_mode='fallback' still returns the FP64
    product."""
    import torch
    import oracle as O
    dev = torch.device("cuda", 0)
    rng = np.random.RandomState(5)
    A, B = rng.randn(96, 5000), rng.randn(5000, 40)
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    case("torch matmul ondevice high (96,5000,40), three calls in a row")
    outs = [ozk.matmul(At, Bt, pipeline="ondevice", accumulation="fused", precision="high")
            for _ in range(3)]
    want = O.matmul_ondevice_a4(A, B, "raise", 4, 1)
    for C in outs:
        assert np.array_equal(C.cpu().numpy(), want)
    A2 = A.copy()
    A2[3, 7] = np.inf
    A2t = torch.from_numpy(A2).to(dev)
    case("torch matmul with Inf input: raise, then fallback")
    with pytest.raises(ValueError, match="NaN or Inf"):
        ozk.matmul(A2t, Bt, pipeline="ondevice", precision="high")
    C = ozk.matmul(A2t, Bt, pipeline="ondevice", precision="high", safe_mode="fallback")
    assert np.array_equal(C.cpu().numpy(), torch.matmul(A2t, Bt).cpu().numpy(), equal_nan=True)


def test_torch_matmul_and_gram_on_a_side_stream(ozk):
    """Under `torch.cuda.stream(s)` the calls run, copy their flags and
    record their events on s; results read after s has drained are exact."""
    import torch
    import oracle as O
    dev = torch.device("cuda", 0)
    rng = np.random.RandomState(6)
    A, B = rng.randn(80, 6000), rng.randn(6000, 72)
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    case("torch matmul and gram on a side stream")
    with torch.cuda.stream(s):
        C = ozk.matmul(At, Bt, pipeline="ondevice", accumulation="fused", precision="high")
        G = ozk.gram(Bt, mode="ozaki", precision="high")
    s.synchronize()
    assert np.array_equal(C.cpu().numpy(), O.matmul_ondevice_a4(A, B, "raise", 4, 1))
    assert np.array_equal(G.cpu().numpy(), ozk.gram(B, mode="ozaki", precision="high"))
