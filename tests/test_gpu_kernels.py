"""GPU parity of the int4 kernels (quantise, dequantise, M=1 GEMV) against the CPU oracle.

Bar: quantised values / scales / zeros and dequantised weights bit-exact; GEMV within the
fp32-accumulation bound of an fp64 brute force, rounded to bf16.
"""
import pytest
import torch

from tests.helpers import log

pytestmark = pytest.mark.gpu

SHAPES = [(3584, 2560), (2560, 2560), (16384, 2560), (2560, 8192), (8, 128), (24, 384)]


def _weights(n, k, seed, kind="normal"):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 0.02)
    if kind == "edge":
        w = w.view(n, k // 128, 128)
        w[0, :] = 0.25                       # constant group -> scale clamp 1e-6
        w[1 % n, 0] = -1.0                   # outlier
        w[-1, -1, :64] = 3.0                 # two-valued group
        w = w.view(n, k)
    return w.to(torch.bfloat16)


@pytest.mark.parametrize("n,k", SHAPES)
def test_quantize_bit_exact(dev, n, k):
    from flint_amd.quantize import quantize_int4, unpack_q, unpack_sz
    from oracle import quant
    for kind in ("normal", "edge"):
        log(f"quantize n={n} k={k} kind={kind}")
        w = _weights(n, k, 1, kind)
        q, sz = quantize_int4(w.to(dev))
        torch.cuda.synchronize()
        qo, so, zo = quant.group_quantize(w)
        assert torch.equal(unpack_q(q).cpu(), qo)
        s, z = unpack_sz(sz)
        assert torch.equal(s.cpu().view(torch.int16), so.view(torch.int16))
        assert torch.equal(z.cpu().view(torch.int16), zo.view(torch.int16))


@pytest.mark.parametrize("matrix_cores", [False, True])
@pytest.mark.parametrize("n,k", SHAPES)
def test_dequant_bit_exact(dev, n, k, matrix_cores):
    """Both device forms of the dequantisation (vector ALUs; 4x4x4 MFMAs lane by lane, the decode
    GEMVs') give the oracle's bits, edge groups (scale clamp, outlier, two values) included."""
    from flint_amd.quantize import quantize_int4, dequantize_int4
    from oracle import quant
    w = _weights(n, k, 2, "edge")
    log(f"dequant n={n} k={k} matrix_cores={matrix_cores}")
    q, sz = quantize_int4(w.to(dev))
    dq = dequantize_int4(q, sz, matrix_cores).cpu()
    ref = quant.dq_linear_weight(w)
    assert torch.equal(dq.view(torch.int16), ref.view(torch.int16))


def test_dequant_mx_extreme_scales(dev):
    """The matrix-core form on hand-set (scale, zero) words across the bf16 range -- tiny and huge
    scales, zeros of both signs and magnitudes that make the fp32 add round -- against the vector
    form, every nibble value in every position."""
    from flint_amd.quantize import dequantize_int4
    g = torch.Generator().manual_seed(11)
    n, k = 64, 512
    q = torch.randint(-2**31, 2**31 - 1, (n, k // 8), generator=g, dtype=torch.int64).to(torch.int32)
    q[0] = 0x76543210
    q[1] = -0x789abcdf   # 0x87654321 as int32
    s = torch.tensor([1e-30, 3e-8, 1e-6, 2.5e-3, 0.02, 1.0, 7.5, 3e4, 1e30], dtype=torch.float32)
    z = torch.tensor([0.0, -0.0, 1e-30, -2.5e-3, 0.6, -1.0, 200.0, -3e4, 1e30], dtype=torch.float32)
    si = torch.randint(0, len(s), (n, k // 128), generator=g)
    zi = torch.randint(0, len(z), (n, k // 128), generator=g)
    sb = s[si].to(torch.bfloat16).view(torch.int16).to(torch.int32) & 0xFFFF
    zb = z[zi].to(torch.bfloat16).view(torch.int16).to(torch.int32) & 0xFFFF
    sz = (sb | (zb << 16)).to(torch.int32)
    a = dequantize_int4(q.to(dev), sz.to(dev), False).cpu()
    b = dequantize_int4(q.to(dev), sz.to(dev), True).cpu()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("n,k", SHAPES)
def test_gemv_vs_fp64(dev, n, k):
    from flint_amd.quantize import quantize_int4, gemv_int4
    from oracle import quant
    w = _weights(n, k, 3)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(k, generator=g).to(torch.bfloat16)
    log(f"gemv n={n} k={k}")
    q, sz = quantize_int4(w.to(dev))
    y = gemv_int4(q, sz, x.to(dev)).cpu()
    dq = quant.dq_linear_weight(w).double()
    ref = dq @ x.double()
    # fp32 accumulation of k products: |err| <= k * 2^-24 * sum|x*w|, plus bf16 output rounding
    bound = k * 2.0 ** -24 * (dq.abs() @ x.double().abs()) + ref.abs() * 2.0 ** -8 + 1e-30
    err = (y.double() - ref).abs()
    assert bool((err <= bound).all()), float((err / bound).max())
    # rounded results agree with the fp64 reference rounded once except at rare rounding ties
    mism = (y != ref.float().to(torch.bfloat16)).float().mean().item()
    log(f"  bf16 mismatch rate vs fp64-rounded: {mism:.2e}")
    assert mism < 2e-3


def test_gemv_matches_oracle_linear(dev):
    """Same contract as the oracle's F.linear on dequantised weights (the reference linear)."""
    from flint_amd.quantize import quantize_int4, gemv_int4
    from oracle import quant
    n, k = 16384, 2560
    w = _weights(n, k, 5)
    x = torch.randn(k, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    q, sz = quantize_int4(w.to(dev))
    y = gemv_int4(q, sz, x.to(dev)).cpu()
    ref = torch.nn.functional.linear(x.view(1, -1), quant.dq_linear_weight(w)).view(-1)
    diff = (y.float() - ref.float()).abs().max().item()
    mism = (y != ref).float().mean().item()
    log(f"gemv vs oracle linear: max|diff|={diff:.3e} mismatch={mism:.2e}")
    assert mism < 2e-3 and diff < 2e-2


GEMM_CASES = [(3584, 2560, 5), (2560, 8192, 8), (16384, 2560, 16), (24, 384, 3), (8, 128, 1),
              (2560, 2560, 2),
              # the second 16-row activation block (tokens 16..31), with N not a multiple of 16
              (3584, 2560, 17), (2568, 8192, 24), (1000, 2560, 32), (24, 384, 32)]


@pytest.mark.parametrize("n,k,m", GEMM_CASES)
def test_gemm_vs_fp64(dev, n, k, m):
    """M-row int4 GEMM on the matrix cores (verify's weight-read-once product): every output within
    the fp32-accumulation bound of the exact product with the bit-exact dequantised weights."""
    from flint_amd.quantize import quantize_int4, gemm_int4
    from oracle import quant
    w = _weights(n, k, 7)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    log(f"gemm n={n} k={k} m={m}")
    q, sz = quantize_int4(w.to(dev))
    y = gemm_int4(q, sz, x.to(dev)).cpu()
    assert y.shape == (m, n)
    dq = quant.dq_linear_weight(w).double()
    ref = x.double() @ dq.t()
    bound = k * 2.0 ** -24 * (x.double().abs() @ dq.abs().t()) + ref.abs() * 2.0 ** -8 + 1e-30
    err = (y.double() - ref).abs()
    assert bool((err <= bound).all()), float((err / bound).max())
    mism = (y != ref.float().to(torch.bfloat16)).float().mean().item()
    log(f"  bf16 mismatch rate vs fp64-rounded: {mism:.2e}")
    assert mism < 2e-3


@pytest.mark.parametrize("m", [8, 32])
def test_gemm_rows_match_gemv(dev, m):
    """Row m of the M-row GEMM equals the M=1 GEMV of x[m] up to fp32 summation order."""
    from flint_amd.quantize import quantize_int4, gemm_int4, gemv_int4
    n, k = 3584, 2560
    w = _weights(n, k, 9)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    q, sz = quantize_int4(w.to(dev))
    y = gemm_int4(q, sz, x.to(dev)).cpu()
    for i in range(m):
        yv = gemv_int4(q, sz, x[i].contiguous().to(dev)).cpu()
        d = (y[i].float() - yv.float()).abs()
        assert float(d.max()) <= float(yv.float().abs().max()) * 2.0 ** -7
        assert float((d > 0).float().mean()) < 2e-3


@pytest.mark.parametrize("lead", [(1,), (8,), (2, 16), (32,), (3, 25)])
def test_weight_only_int4_linear(dev, lead):
    """WeightOnlyInt4Linear (the drop-in for reference engine/quantize.py:483-525) at M = 1
    (the GEMV), M up to 32 (one GEMM launch, leading dimensions flattened) and M = 75 (three
    launches of up to 32 rows, as gpt-fast's prefill passes a whole prompt) against the oracle's
    linear on the dequantised weights; its buffers hold the quantised values exactly."""
    from flint_amd.quantize import WeightOnlyInt4Linear, unpack_q, unpack_sz
    from oracle import quant
    n, k = 2560, 2560
    w = _weights(n, k, 12)
    mod = WeightOnlyInt4Linear.from_float(w.to(dev))
    qo, so, zo = quant.group_quantize(w)
    assert torch.equal(unpack_q(mod.weight).cpu(), qo)
    s, z = unpack_sz(mod.scales_and_zeros)
    assert torch.equal(s.cpu().view(torch.int16), so.view(torch.int16))
    assert torch.equal(z.cpu().view(torch.int16), zo.view(torch.int16))
    g = torch.Generator().manual_seed(13)
    x = torch.randn(*lead, k, generator=g).to(torch.bfloat16)
    y = mod(x.to(dev)).cpu()
    assert y.shape == (*lead, n) and y.dtype == torch.bfloat16
    ref = torch.nn.functional.linear(x.reshape(-1, k), quant.dq_linear_weight(w)).view(*lead, n)
    diff = (y.float() - ref.float()).abs().max().item()
    mism = (y != ref).float().mean().item()
    log(f"WeightOnlyInt4Linear lead={lead}: max|diff|={diff:.3e} mismatch={mism:.2e}")
    assert mism < 2e-3 and diff <= 2.0 ** -7 * float(ref.float().abs().max())
    with pytest.raises(Exception):
        mod(torch.zeros(4, k + 128, dtype=torch.bfloat16, device=dev))  # wrong inner dimension


def test_scales_and_zeros_gptfast_layout(dev):
    """scales_and_zeros_gptfast gives gpt-fast's [K/128, N, 2] bf16 tensor
    (reference engine/quantize.py:79-93 pack_scales_and_zeros) of the same values the oracle
    packs."""
    from flint_amd.quantize import quantize_int4, scales_and_zeros_gptfast
    from oracle import quant
    n, k = 384, 1024
    w = _weights(n, k, 14, "edge")
    q, sz = quantize_int4(w.to(dev))
    got = scales_and_zeros_gptfast(sz).cpu()
    _, so, zo = quant.group_quantize(w)
    ref = quant.pack_scales_and_zeros(so, zo)
    assert got.shape == (k // 128, n, 2) and got.dtype == torch.bfloat16
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    # the reference's definition: entry [g, n] = (scale, zero) of row n, group g
    for g, r in ((0, 0), (3, 17), (7, n - 1)):
        assert got[g, r, 0].view(torch.int16) == so[r, g].view(torch.int16)
        assert got[g, r, 1].view(torch.int16) == zo[r, g].view(torch.int16)


TILED_SHAPES = [(3584, 2560), (16384, 2560), (2560, 8192), (16, 128), (48, 384), (32, 16384)]


def _tiled(q, n, k):
    from flint_amd import _lib
    qt = torch.empty(n // 16, k // 128, 64, 4, dtype=torch.int32, device=q.device)
    _lib.call("fl_tile_int4", _lib.ptr(q), _lib.ptr(qt), n, k, _lib.stream_ptr())
    return qt


@pytest.mark.parametrize("n,k", TILED_SHAPES)
def test_tiled_dequant_bit_exact(dev, n, k):
    """The matrix-core dequantisation (fl_tile_int4 + fl_dequant_int4_tiled: D1 = (128+q) diag(s)
    - 136 s, round, D2 = I a + z, round) gives gpt-fast's bf16(bf16((q-8) s) + z) bit for bit,
    edge groups included (constant group, outlier, two-valued group)."""
    from flint_amd import _lib
    from flint_amd.quantize import quantize_int4
    from oracle import quant
    w = _weights(n, k, 21, "edge")
    log(f"tiled dequant n={n} k={k}")
    q, sz = quantize_int4(w.to(dev))
    qt = _tiled(q, n, k)
    out = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
    _lib.call("fl_dequant_int4_tiled", _lib.ptr(qt), _lib.ptr(sz), _lib.ptr(out), n, k, _lib.stream_ptr())
    ref = quant.dq_linear_weight(w)
    got = out.cpu()
    bad = (got.view(torch.int16) != ref.view(torch.int16))
    if bool(bad.any()):
        idx = bad.nonzero()[:12].tolist()
        rows = bad.nonzero()[:, 0] % 16
        cols = bad.nonzero()[:, 1] % 128
        log(f"  {int(bad.sum())} of {bad.numel()} differ; rows mod 16 {torch.bincount(rows, minlength=16).tolist()}; "
            f"cols mod 16 {torch.bincount(cols % 16, minlength=16).tolist()}; cols // 16 {torch.bincount(cols // 16, minlength=8).tolist()}")
        for r, c in idx:
            log(f"  [{r},{c}] got {float(got[r, c])} want {float(ref[r, c])}")
    assert not bool(bad.any())


@pytest.mark.parametrize("n,k", TILED_SHAPES)
def test_tiled_gemv_vs_fp64(dev, n, k):
    """The matrix-core GEMV within the fp32-accumulation bound of the exact product, and equal to
    the row-layout GEMV up to fp32 summation order."""
    from flint_amd import _lib
    from flint_amd.quantize import quantize_int4, gemv_int4
    from oracle import quant
    w = _weights(n, k, 22)
    x = torch.randn(k, generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    log(f"tiled gemv n={n} k={k}")
    q, sz = quantize_int4(w.to(dev))
    qt = _tiled(q, n, k)
    y = torch.empty(n, dtype=torch.bfloat16, device=dev)
    _lib.call("fl_gemv_int4_tiled", _lib.ptr(qt), _lib.ptr(sz), _lib.ptr(x.to(dev)), _lib.ptr(y), n, k,
              _lib.stream_ptr())
    y = y.cpu()
    dq = quant.dq_linear_weight(w).double()
    ref = dq @ x.double()
    bound = k * 2.0 ** -24 * (dq.abs() @ x.double().abs()) + ref.abs() * 2.0 ** -8 + 1e-30
    err = (y.double() - ref).abs()
    assert bool((err <= bound).all()), float((err / bound).max())
    mism = (y != ref.float().to(torch.bfloat16)).float().mean().item()
    yr = gemv_int4(q, sz, x.to(dev)).cpu()
    log(f"  bf16 mismatch vs fp64-rounded {mism:.2e}, vs row-layout GEMV {(y != yr).float().mean().item():.2e}")
    assert mism < 2e-3
