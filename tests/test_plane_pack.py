"""The host-side packing of caller-held BF16 slices into the library's plane
layout (pallas_gemm_accum._pack_bf16_planes), decoded with the byte-address
rule of include/ozaki_amd.h: byte b of line r of a plane with L lines lies at
((b / 64) * L + r) * 64 + 16 * (((b % 64) / 16) ^ s(r)) + b % 16,
s(r) = (((r & 15) >> 1) ^ ((r & 15) >> 2)) & 3."""

import numpy as np
import pytest

from ozaki_jax_amd.pallas_gemm_accum import _make_pair_schedule, _pack_bf16_planes


def _decode(plane_bytes, L, nbytes_per_line):
    out = np.zeros((L, nbytes_per_line), np.uint8)
    for r in range(L):
        s = (((r & 15) >> 1) ^ ((r & 15) >> 2)) & 3
        for b in range(nbytes_per_line):
            out[r, b] = plane_bytes[((b // 64) * L + r) * 64 + 16 * (((b % 64) // 16) ^ s) + b % 16]
    return out


@pytest.mark.parametrize("shape", [(2, 3, 5), (1, 70, 100), (3, 64, 64)])
def test_pack_matches_the_header_layout(shape):
    rng = np.random.RandomState(sum(shape))
    vals = (rng.randint(-128, 129, size=shape) * 2.0 ** rng.randint(-20, 20)).astype(np.float32)
    packed, Lp = _pack_bf16_planes(vals)
    n, L, K = shape
    assert Lp % 64 == 0 and packed.shape[1] == Lp and packed.shape[2] % 64 == 0
    for p in range(n):
        raw = np.ascontiguousarray(packed[p]).view(np.uint8).reshape(-1)
        dec = _decode(raw, Lp, packed.shape[2] * 2).view(np.uint16)
        assert np.array_equal(dec[:L, :K], (vals[p].view(np.uint32) >> 16).astype(np.uint16))
        assert not dec[L:].any() and not dec[:, K:].any()


def test_pack_rejects_values_that_are_not_bf16():
    with pytest.raises(ValueError, match="BF16-exact"):
        _pack_bf16_planes(np.full((1, 2, 2), 1.0 + 2.0 ** -20, np.float32))


def test_pair_schedule_matches_the_reference_test():
    """test_pallas_fused.py:26-50 of the reference, on this mirror."""
    pair_a, pair_b, n_pairs, groups, bb = _make_pair_schedule(4, 1)
    assert n_pairs == 24 and bb == (4, 8, 9)
    for idx in range(16):
        assert (pair_a[idx], pair_b[idx]) == divmod(idx, 4)
    assert all(pair_a[i] == i - 16 and pair_b[i] == 4 for i in range(16, 20))
    assert all(pair_a[i] == 4 and pair_b[i] == i - 20 for i in range(20, 24))
    assert [len(p) for _, p in groups] == [4] * 4 + [1] * 4 + [4]


def test_device_array_sizes():
    """Bytes a NumPy-family device array covers: 2-D rows with a leading
    dimension, other ranks contiguous (a stand-in block: no device needed)."""
    from ozaki_jax_amd._hip import DeviceArray

    class Block:
        ptr = 4096

    assert DeviceArray((3, 4, 5), np.uint16, block=Block()).nbytes == 120
    assert DeviceArray((4, 5), np.float64, ld=8, block=Block()).nbytes == (3 * 8 + 5) * 8
    assert DeviceArray((7,), np.int32, block=Block()).nbytes == 28
    assert DeviceArray((0, 5), np.float64, block=Block()).nbytes == 0
    col = DeviceArray((6,), np.float64, block=Block()).column()
    assert col.shape == (6, 1) and col.nbytes == 48 and col.stride(0) == 1
