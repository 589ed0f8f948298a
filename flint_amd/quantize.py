"""Host side of the int4 weight path: quantise / dequantise / M=1 and M=k GEMV, all on the GPU
through the C ABI, plus a drop-in for gpt-fast's WeightOnlyInt4Linear.

Mirrors reference engine/quantize.py:359-525 (prepare_int4_weight_and_scales_and_zeros,
linear_forward_int4, WeightOnlyInt4Linear): same groupsize (128), same quantised values,
same dequantised bf16 values; the packed layout is this library's own (see include/flint_amd.h).
"""
import torch

from . import _lib

GROUP = _lib.GROUP


def _check_dev(t, dtype, name):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def quantize_int4(w, q=None, sz=None):
    """Quantise a bf16 [N, K] device matrix group-wise (128) to (q int32 [N, K/8], sz int32 [N, K/128])."""
    _check_dev(w, torch.bfloat16, "w")
    n, k = w.shape
    if k % GROUP:
        raise ValueError("K must be a multiple of 128")
    if q is None:
        q = torch.empty(n, k // 8, dtype=torch.int32, device=w.device)
    if sz is None:
        sz = torch.empty(n, k // GROUP, dtype=torch.int32, device=w.device)
    _lib.call("fl_quantize_int4", _lib.ptr(w), _lib.ptr(q), _lib.ptr(sz), n, k, _lib.stream_ptr())
    return q, sz


def dequantize_int4(q, sz, matrix_cores=False):
    """Bit-exact bf16 [N, K] dequantisation through the kernels' own device routine: the vector-ALU
    form (fl_gemm_int4's) or, with matrix_cores, the lane-by-lane MFMA form of the decode GEMVs and
    fl_gemv_int4."""
    _check_dev(q, torch.int32, "q")
    _check_dev(sz, torch.int32, "sz")
    n, k = q.shape[0], q.shape[1] * 8
    out = torch.empty(n, k, dtype=torch.bfloat16, device=q.device)
    _lib.call("fl_dequant_int4_mx" if matrix_cores else "fl_dequant_int4", _lib.ptr(q), _lib.ptr(sz),
              _lib.ptr(out), n, k, _lib.stream_ptr())
    return out


def tile_int4(q, qt=None):
    """The tiled layout (fl_tile_int4) of a row-layout int4 matrix q [..., N, K/8] (N % 16 == 0;
    leading dims are stacked rows): same shape and dtype, 1 KB per 16 rows x 128-group unit."""
    _check_dev(q, torch.int32, "q")
    k = q.shape[-1] * 8
    n = q.numel() // q.shape[-1]
    if n % 16:
        raise ValueError("tile_int4: the stacked row count must be a multiple of 16")
    if qt is None:
        qt = torch.empty_like(q)
    elif qt.shape != q.shape or qt.dtype != torch.int32 or not qt.is_contiguous():
        raise ValueError("tile_int4: qt must be a contiguous int32 tensor shaped like q")
    _lib.call("fl_tile_int4", _lib.ptr(q), _lib.ptr(qt), n, k, _lib.stream_ptr())
    return qt


def gemv_int4(q, sz, x, y=None):
    """y[N] = bf16(x[K] . dq[N,K]^T) with fp32 accumulation (M = 1)."""
    _check_dev(q, torch.int32, "q")
    _check_dev(sz, torch.int32, "sz")
    _check_dev(x, torch.bfloat16, "x")
    n, k = q.shape[0], q.shape[1] * 8
    if x.numel() != k:
        raise ValueError(f"x has {x.numel()} elements, expected {k}")
    if y is None:
        y = torch.empty(n, dtype=torch.bfloat16, device=q.device)
    _lib.call("fl_gemv_int4", _lib.ptr(q), _lib.ptr(sz), _lib.ptr(x), _lib.ptr(y), n, k,
              _lib.stream_ptr())
    return y


def gemm_int4(q, sz, x, y=None):
    """Y[M,N] = bf16(X[M,K] . dq[N,K]^T) for any M: blocks of up to 32 rows (FL_MAX_VERIFY), each
    one fl_gemm_int4 launch that reads the weights once for all of its rows."""
    _check_dev(q, torch.int32, "q")
    _check_dev(sz, torch.int32, "sz")
    _check_dev(x, torch.bfloat16, "x")
    n, k = q.shape[0], q.shape[1] * 8
    m = x.shape[0]
    if x.shape[1] != k:
        raise ValueError("x inner dimension mismatch")
    if y is None:
        y = torch.empty(m, n, dtype=torch.bfloat16, device=q.device)
    if m > 0 and (y.shape != (m, n) or not y.is_contiguous()):
        raise ValueError("y must be a contiguous [M, N] tensor")
    for r0 in range(0, m, _lib.MAX_VERIFY):
        mb = min(_lib.MAX_VERIFY, m - r0)
        _lib.call("fl_gemm_int4", _lib.ptr(q), _lib.ptr(sz), _lib.ptr(x[r0:]), _lib.ptr(y[r0:]), mb, n, k,
                  _lib.stream_ptr())
    return y


# bit position of element e (0..7) inside its packed word: element 2i at 4i, 2i+1 at 16+4i
NIBBLE_SHIFT = [0, 16, 4, 20, 8, 24, 12, 28]


def unpack_q(q):
    """int32 [N, K/8] packed words -> int32 [N, K] values in [0, 15] (host-side inspection)."""
    shifts = torch.tensor(NIBBLE_SHIFT, device=q.device, dtype=torch.int32)
    v = (q.unsqueeze(-1) >> shifts) & 0xF
    return v.reshape(q.shape[0], q.shape[1] * 8)


def pack_q(vals):
    """int32 [N, K] values in [0, 15] -> int32 [N, K/8] packed words (inverse of unpack_q)."""
    n, k = vals.shape
    v = vals.to(torch.int64).view(n, k // 8, 8)
    shifts = torch.tensor(NIBBLE_SHIFT, device=vals.device, dtype=torch.int64)
    words = (v << shifts).sum(-1)
    return torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)


def unpack_sz(sz):
    """int32 [N, K/128] -> (scales bf16 [N, K/128], zeros bf16 [N, K/128])."""
    s = (sz & 0xFFFF).to(torch.int16).view(torch.bfloat16)
    z = ((sz >> 16) & 0xFFFF).to(torch.int16).view(torch.bfloat16)
    return s, z


def scales_and_zeros_gptfast(sz):
    """Our [N, K/128] scale/zero words -> gpt-fast's packed [K/128, N, 2] bf16 layout
    (reference engine/quantize.py:79-93 pack_scales_and_zeros)."""
    s, z = unpack_sz(sz)
    return torch.stack([s, z], dim=-1).transpose(0, 1).contiguous()


class WeightOnlyInt4Linear(torch.nn.Module):
    """Drop-in for reference engine/quantize.py:483-525 (groupsize 128), on the HIP GEMVs.

    forward(x [..., K] bf16) -> [..., N] bf16; M = prod(leading dims) <= 32 rows per call
    (one weight read for all rows), as in decode and speculative verify; more rows raise.
    """

    def __init__(self, in_features, out_features, bias=False, device=None, groupsize=GROUP):
        super().__init__()
        if bias:
            raise ValueError("require bias=False")
        if groupsize != GROUP:
            raise ValueError("groupsize must be 128")
        if in_features % GROUP:
            raise ValueError("in_features must be a multiple of 128")
        self.in_features, self.out_features = in_features, out_features
        self.register_buffer("weight", torch.zeros(out_features, in_features // 8,
                                                   dtype=torch.int32, device=device))
        self.register_buffer("scales_and_zeros", torch.zeros(out_features, in_features // GROUP,
                                                             dtype=torch.int32, device=device))

    @classmethod
    def from_float(cls, w):
        m = cls(w.shape[1], w.shape[0], device=w.device)
        quantize_int4(w.to(torch.bfloat16).contiguous(), m.weight, m.scales_and_zeros)
        return m

    def forward(self, x):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).to(torch.bfloat16).contiguous()
        if x2.shape[0] == 1:
            y = gemv_int4(self.weight, self.scales_and_zeros, x2.view(-1)).view(1, -1)
        else:
            y = gemm_int4(self.weight, self.scales_and_zeros, x2)
        return y.view(*shape[:-1], self.out_features)
