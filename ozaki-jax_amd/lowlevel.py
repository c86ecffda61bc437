"""Stage-level access to the C ABI (extraction planes, slice GEMM, per-pair
products) on device tensors.  Used by the parity tests to check each stage of
the pipeline separately, and by callers that keep slices resident (e.g. to
reuse one operand's extraction across several products)."""

from . import _device as D
from . import _lib

PIPE_ONDEVICE = _lib.PIPE_ONDEVICE
PIPE_HOST = _lib.PIPE_HOST
ORDER_2SUM = _lib.ORDER_2SUM
ORDER_BLOCK64 = _lib.ORDER_BLOCK64
ORDER_HOST_JAX = _lib.ORDER_HOST_JAX
ORDER_HOST_NP = _lib.ORDER_HOST_NP


CHUNK_BYTES = 64


def unit_swizzle(line):
    """Stored position of logical 16-byte unit 0 of `line` (XOR key)."""
    r = line & 15
    return ((r >> 1) ^ (r >> 2)) & 3


class Planes:
    """Slice planes of one operand on the device.

    s: (planes, lines_pad, ld) storage of int16 BF16 bit patterns, or of int8
    grid counts q = slice * 2^(24 - rho) stored as q + offset (offset =
    2^(25 - rho) - 1) when `rho` is set (INT8 format).
    The bytes of a plane are chunk-major (64-byte chunks of k, chunk c of
    every line together, the four 16-byte units of a line's chunk stored in
    the order u ^ unit_swizzle(line)); grid() returns the plain
    (planes, lines_pad, ld) arrangement.
    e: int32 (planes, lines_pad) exponents; sums: int32 (planes, lines_pad)
    line sums of q (INT8 only); lines / length: logical sizes.
    """

    def __init__(self, s, e, lines, length, flags, rho=None, sums=None):
        self.s, self.e, self.lines, self.length, self.flags = s, e, lines, length, flags
        self.rho = rho
        self.sums = sums

    @property
    def i8(self):
        return self.rho is not None

    @property
    def offset(self):
        """The INT8 format's offset 2^(25 - rho) - 1."""
        return (1 << (25 - self.rho)) - 1

    def counts(self):
        """INT8 grid counts q as int32 (planes, lines_pad, ld) (device)."""
        return self.grid().to(D.torch.int32) - self.offset

    def _sums_ptr(self):
        return self.sums.data_ptr() if self.sums is not None else None

    def grid(self):
        """Plane elements as (planes, lines_pad, ld), line-major (device)."""
        torch = D.torch
        P, L, ld = self.s.shape
        eb = self.s.element_size()
        nch = ld * eb // CHUNK_BYTES
        raw = self.s.contiguous().view(-1).view(torch.uint8).reshape(P, nch, L, 4, 16)
        r = torch.arange(L, device=raw.device)
        stored = torch.arange(4, device=raw.device)[None, :] ^ unit_swizzle(r)[:, None]
        raw = raw[:, :, r[:, None], stored, :]
        raw = raw.permute(0, 2, 1, 3, 4).contiguous().reshape(P, L, nch * CHUNK_BYTES)
        return raw.view(self.s.dtype).reshape(P, L, ld)

    def values(self):
        """float32 (planes, lines, length) slice values (device)."""
        g = self.grid()
        if self.i8:
            v = (g.to(D.torch.int32) - self.offset).to(D.torch.float32) * 2.0 ** (self.rho - 24)
        else:
            v = (g.to(D.torch.int32) << 16).view(D.torch.float32)
        return v[:, :self.lines, :self.length]

    def exponents(self):
        return self.e[:, :self.lines]

    def nonfinite(self):
        return D.read_flags(self.flags) & _lib.OZK_FLAG_NONFINITE


def extract(X, by_cols, rho, n0, n1=0, f64=False, i8=False):
    """Run ozk_extract_f32 (n0 hi slices, n1 lo slices), ozk_extract_f32_i8
    (the same with INT8 planes) or ozk_extract_f64 (n0 slices) on X (any 2-D
    array; copied to the device as float64)."""
    lib = _lib.load()
    dev = D.require_gpu()
    Xt = D.to_device_f64(X, dev)
    rows, cols = Xt.shape
    lines, length = (cols, rows) if by_cols else (rows, cols)
    planes = n0 if f64 else n0 + n1
    s = D.torch.zeros((planes, lib.ozk_slice_lines(max(lines, 1)),
                       lib.ozk_slice_ld(max(length, 1))),
                      dtype=D.torch.int8 if i8 else D.torch.int16, device=dev)
    e = D.torch.zeros((planes, lib.ozk_slice_lines(max(lines, 1))),
                      dtype=D.torch.int32, device=dev)
    sums = D.torch.zeros_like(e) if i8 else None
    flags = None

    def once():
        nonlocal flags
        flags = D.new_flags(dev)  # the extraction entry points OR into the word
        wsb = lib.ozk_extract_workspace_bytes(rows, cols, int(by_cols))
        ws = D.workspace(wsb, dev)
        if f64:
            rc = lib.ozk_extract_f64(Xt.data_ptr(), rows, cols, D.ld_of(Xt),
                                     int(by_cols), rho, n0, s.data_ptr(),
                                     e.data_ptr(), flags.data_ptr(), ws.data_ptr(),
                                     wsb, D.stream_handle())
        elif i8:
            rc = lib.ozk_extract_f32_i8(Xt.data_ptr(), rows, cols, D.ld_of(Xt), int(by_cols),
                                        rho, n0, n1, s.data_ptr(), e.data_ptr(),
                                        sums.data_ptr(), flags.data_ptr(), ws.data_ptr(),
                                        wsb, D.stream_handle())
        else:
            rc = lib.ozk_extract_f32(Xt.data_ptr(), rows, cols, D.ld_of(Xt), int(by_cols),
                                     rho, n0, n1, s.data_ptr(), e.data_ptr(),
                                     flags.data_ptr(), ws.data_ptr(), wsb, D.stream_handle())
        _lib.check(rc)
        return D.read_flags(flags)

    _lib.with_gang_retry(once)
    return Planes(s, e, lines, length, flags, rho if i8 else None, sums)


def gemm(a, b, pipeline, n_hi, n_lo, order, workspace_bytes=None):
    """ozk_gemm on two Planes (a: rows of A, b: columns of B) -> C (N, M).
    workspace_bytes: at least ozk_gemm_workspace_bytes (the default); what
    lies beyond it holds the partial sums of a K-split tail."""
    lib = _lib.load()
    dev = a.s.device
    N, M, K = a.lines, b.lines, a.length
    C = D.torch.empty((N, M), dtype=D.torch.float64, device=dev)
    wsb = lib.ozk_gemm_workspace_bytes(N, M, pipeline, n_hi, n_lo, order)
    if workspace_bytes is not None:
        wsb = max(wsb, int(workspace_bytes))
    ws = D.workspace(wsb, dev)
    if a.i8:
        rc = lib.ozk_gemm_i8(a.s.data_ptr(), a.e.data_ptr(), a._sums_ptr(), b.s.data_ptr(),
                             b.e.data_ptr(), b._sums_ptr(), N, M, K, a.rho, n_hi, n_lo, order,
                             C.data_ptr(), max(M, 1), ws.data_ptr(), wsb,
                             D.stream_handle())
    else:
        rc = lib.ozk_gemm(a.s.data_ptr(), a.e.data_ptr(), b.s.data_ptr(),
                          b.e.data_ptr(), N, M, K, pipeline, n_hi, n_lo, order,
                          C.data_ptr(), max(M, 1), ws.data_ptr(), wsb,
                          D.stream_handle())
    _lib.check(rc)
    return C


def gemm_pair(a, b, n_hi, n_lo):
    """ozk_gemm_2sum_pair on two Planes -> (C_hi, C_lo) float32 (N, M)."""
    lib = _lib.load()
    dev = a.s.device
    N, M, K = a.lines, b.lines, a.length
    C_hi = D.torch.empty((N, M), dtype=D.torch.float32, device=dev)
    C_lo = D.torch.empty((N, M), dtype=D.torch.float32, device=dev)
    wsb = lib.ozk_gemm_workspace_bytes(N, M, PIPE_ONDEVICE, n_hi, n_lo, ORDER_2SUM)
    ws = D.workspace(wsb, dev)
    _lib.check(lib.ozk_gemm_2sum_pair(a.s.data_ptr(), a.e.data_ptr(), a._sums_ptr(),
                                      b.s.data_ptr(), b.e.data_ptr(), b._sums_ptr(),
                                      N, M, K, 1 if a.i8 else 2,
                                      a.rho or 0, n_hi, n_lo, C_hi.data_ptr(),
                                      C_lo.data_ptr(), max(M, 1), ws.data_ptr(), wsb,
                                      D.stream_handle()))
    return C_hi, C_lo


def slice_products(a, b, pipeline, n_hi, n_lo):
    """ozk_slice_products -> float32 (n_pairs, N, M) device tensor."""
    lib = _lib.load()
    dev = a.s.device
    N, M, K = a.lines, b.lines, a.length
    npairs = _lib.check(lib.ozk_pair_count(pipeline, n_hi, n_lo))
    P = D.torch.zeros((npairs, N, M), dtype=D.torch.float32, device=dev)
    if a.i8:
        rc = lib.ozk_slice_products_i8(a.s.data_ptr(), a._sums_ptr(), b.s.data_ptr(),
                                       b._sums_ptr(), N, M, K,
                                       a.rho, n_hi, n_lo, P.data_ptr(),
                                       max(M, 1), D.stream_handle())
    else:
        rc = lib.ozk_slice_products(a.s.data_ptr(), b.s.data_ptr(), N, M, K,
                                    pipeline, n_hi, n_lo, P.data_ptr(),
                                    max(M, 1), D.stream_handle())
    _lib.check(rc)
    return P


def probe_mfma_layout():
    """Accumulator registers after the layout-probe MFMAs, as int32 arrays
    (32x32x16 BF16: (64 lanes, 16 regs), values row + 64 col; 16x16x32 BF16:
    (64, 4), row + 64 col; 16x16x64 INT8: (64, 4), row + 16 col; 32x32x32
    INT8: (64 lanes, 16 regs), row + 64 col)."""
    lib = _lib.load()
    dev = D.require_gpu()
    out = D.torch.zeros(2 * 64 * 16 + 2 * 64 * 4, dtype=D.torch.int32, device=dev)
    _lib.check(lib.ozk_probe_mfma_layout(out.data_ptr(), D.stream_handle()))
    o = out.cpu().numpy()
    return (o[:1024].reshape(64, 16), o[1024:1280].reshape(64, 4),
            o[1280:1536].reshape(64, 4), o[1536:].reshape(64, 16))
