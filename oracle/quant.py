"""gpt-fast int4 group quantisation restated on the CPU (test infrastructure only).

Every operation is a torch bf16 tensor op in the reference, i.e. computed in fp32 and rounded
to bf16; the restatement keeps the same operations in the same order so the rounding points
match. Group size 128, 4 bits, asymmetric (scale, zero) per (row, group).
"""
import torch

N_BIT = 4
GROUP = 128


def group_qparams(w, groupsize=GROUP):
    """(scales, zeros) bf16 [N, K/G] of a bf16 [N, K] matrix.
    Restates reference engine/quantize.py:58-76 get_group_qparams."""
    assert w.dtype == torch.bfloat16 and w.dim() == 2 and w.shape[1] % groupsize == 0
    g = w.reshape(-1, groupsize)
    hi = g.amax(dim=1, keepdim=True)
    lo = g.amin(dim=1, keepdim=True)
    levels = 2 ** N_BIT - 1
    scales = (hi - lo).clamp(min=1e-6) / levels
    zeros = lo + scales * (2 ** (N_BIT - 1))
    return scales.reshape(w.shape[0], -1), zeros.reshape(w.shape[0], -1)


def quantize_from_qparams(w, scales, zeros, groupsize=GROUP):
    """int32 [N, K] in [0, 15]. Restates reference engine/quantize.py:102-128."""
    g = w.reshape(-1, groupsize)
    s = scales.reshape(-1, 1)
    lo = zeros.reshape(-1, 1) - s * (2 ** (N_BIT - 1))
    q = g.sub(lo).div(s).round().clamp_(0, 2 ** N_BIT - 1)
    return q.to(torch.int32).reshape(w.shape)


def group_quantize(w, groupsize=GROUP):
    """(q int32 [N,K], scales bf16 [N,K/G], zeros bf16 [N,K/G]).
    Restates reference engine/quantize.py:131-135 group_quantize_tensor (before packing)."""
    s, z = group_qparams(w, groupsize)
    return quantize_from_qparams(w, s, z, groupsize), s, z


def group_dequantize(q, scales, zeros, groupsize=GROUP):
    """bf16 [N, K] = bf16(bf16((q - 8) * s) + z).
    Restates reference engine/quantize.py:138-155 group_dequantize_tensor_from_qparams."""
    g = q.reshape(-1, groupsize)
    out = g.sub(2 ** (N_BIT - 1)).mul(scales.reshape(-1, 1)).add(zeros.reshape(-1, 1))
    return out.reshape(q.shape)


def pack_scales_and_zeros(scales, zeros):
    """[K/G, N, 2] bf16. Restates reference engine/quantize.py:79-93."""
    return torch.stack([scales, zeros], dim=-1).transpose(0, 1).contiguous()


def dq_linear_weight(w):
    """Quantise then dequantise: the bf16 weight every int4 linear of the reference multiplies by."""
    q, s, z = group_quantize(w)
    return group_dequantize(q, s, z)
