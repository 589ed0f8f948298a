"""Pins of the CPU oracle itself (no GPU): library routines, closed forms, invariants, identities.

Each check is chosen so that a plausible mistake in the restatement (wrong zero offset, sign,
scale layout, rounding point, pair order, head mapping) fails it.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import quant
from oracle import model as om


def _w(n, k, seed, std=0.02):
    return (torch.randn(n, k, generator=torch.Generator().manual_seed(seed)) * std).to(torch.bfloat16)


# ---------------------------------------------------------------- quantisation

def test_quant_range_and_roundtrip_bound():
    w = _w(64, 512, 0)
    q, s, z = quant.group_quantize(w)
    assert q.dtype == torch.int32 and int(q.min()) >= 0 and int(q.max()) <= 15
    dq = quant.group_dequantize(q, s, z).float()
    # |w - dq| <= scale/2 (nearest level) + two bf16 roundings of dq and one of the division
    sc = s.float().repeat_interleave(128, dim=1)
    err = (w.float() - dq).abs()
    assert bool((err <= 0.5 * sc + 2.0 ** -7 * dq.abs() + 0.05 * sc).all())
    # levels span the group: q hits 0 and 15 in (almost) every group
    g = q.view(-1, 128)
    assert float(((g.min(1).values == 0) & (g.max(1).values == 15)).float().mean()) > 0.9


def test_quant_special_groups():
    w = torch.zeros(2, 256, dtype=torch.bfloat16)
    w[0, :128] = 0.25                         # constant group: scale clamps at bf16(1e-6)/15
    w[0, 128:] = torch.tensor([-1.0, 3.0]).repeat(64).to(torch.bfloat16)   # two values
    w[1] = _w(1, 256, 3)[0]
    q, s, z = quant.group_quantize(w)
    clamp = torch.tensor(1e-6).to(torch.bfloat16)
    assert s[0, 0] == (clamp / 15)
    dq = quant.group_dequantize(q, s, z)
    assert torch.allclose(dq[0, :128].float(), torch.full((128,), 0.25), atol=1e-5)
    assert set(q[0, 128:].tolist()) == {0, 15}
    assert torch.allclose(dq[0, 128:].float(), w[0, 128:].float(), rtol=1e-2)


def test_dequant_matches_torch_int4_cpu_library_kernel():
    """aten::_weight_int4pack_mm_for_cpu (an independent library implementation of the int4
    linear, scales_and_zeros in the reference's [K/G, N, 2] layout) agrees with
    F.linear(x, oracle dequant) to within the dequant rounding."""
    n, k = 256, 1024
    w = _w(n, k, 1)
    q, s, z = quant.group_quantize(w)
    wp = torch.ops.aten._convert_weight_to_int4pack_for_cpu(q, 8)
    sz = quant.pack_scales_and_zeros(s, z)
    x = torch.randn(3, k, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    lib = torch.ops.aten._weight_int4pack_mm_for_cpu(x, wp, 128, sz).float()
    ref = F.linear(x, quant.group_dequantize(q, s, z)).float()
    scale = (x.float().abs() @ w.float().abs().T)
    # per-element dq rounding error <= 2^-8 relative; plus bf16 output rounding of both sides
    assert bool(((lib - ref).abs() <= 2.0 ** -8 * scale + 2.0 ** -7 * ref.abs() + 1e-4).all())
    # a wrong zero offset (q-7 instead of q-8) would be caught:
    bad = F.linear(x, (q.view(-1, 128) - 7).to(torch.bfloat16).mul(s.reshape(-1, 1))
                   .add(z.reshape(-1, 1)).reshape(n, k)).float()
    assert float((lib - bad).abs().max()) > 10 * float((lib - ref).abs().max())


def test_dequant_two_rounding_points():
    """bf16((q-8)*s) is rounded before adding z (int32.mul(bf16) is a bf16 op)."""
    q = torch.tensor([[11] * 128], dtype=torch.int32)      # q-8 = 3
    s = torch.tensor([[1.0078125]], dtype=torch.bfloat16)  # 1 + 2^-7: 3*s needs 9 bits
    z = torch.tensor([[0.0]], dtype=torch.bfloat16)
    dq = quant.group_dequantize(q, s, z)
    assert float(dq[0, 0]) == float(torch.tensor(3 * 1.0078125).to(torch.bfloat16))
    z2 = torch.tensor([[2.0 ** -6]], dtype=torch.bfloat16)
    dq2 = quant.group_dequantize(q, s, z2)
    exact_single = torch.tensor(3 * 1.0078125 + 2.0 ** -6).to(torch.bfloat16)
    double = torch.tensor(float(torch.tensor(3 * 1.0078125).to(torch.bfloat16)) + 2.0 ** -6).to(torch.bfloat16)
    assert float(dq2[0, 0]) == float(double)
    assert float(double) != float(exact_single)  # the case distinguishes the two roundings


# ---------------------------------------------------------------- RoPE

def test_rope_table_closed_form():
    t = om.freqs_cis(16, 64, 10000)
    assert t.shape == (16, 32, 2) and t.dtype == torch.bfloat16
    for p in (0, 3, 15):
        for i in (0, 5, 31):
            ang = p * 10000 ** (-2 * i / 64)
            assert abs(float(t[p, i, 0]) - math.cos(ang)) <= 2 ** -8
            assert abs(float(t[p, i, 1]) - math.sin(ang)) <= 2 ** -8


def test_rope_neox_equals_interleaved_on_permuted_rows():
    """NEOX half-split on HF-ordered rows == gpt-fast interleaved RoPE on rows permuted as
    convert_hf_checkpoint.permute does (reference engine/scripts/convert_hf_checkpoint.py:75-81)."""
    H, hd, M = 6, 64, 5
    x = torch.randn(M, H, hd, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    table = om.freqs_cis(64, hd, 10000)
    rows = table[torch.tensor([0, 1, 7, 33, 63])]
    perm = om.hf_to_interleaved_perm(H, hd)
    neox = om.rope_neox(x, rows).reshape(M, -1)
    inter = om.rope_interleaved(x.reshape(M, -1)[:, perm].reshape(M, H, hd), rows).reshape(M, -1)
    assert torch.equal(neox[:, perm], inter)
    # pos 0 is the identity
    assert torch.equal(om.rope_neox(x[:1], table[:1]), x[:1])


def test_rope_relative_position_property():
    hd = 64
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 1, hd, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 1, hd, generator=g).to(torch.bfloat16)
    table = om.freqs_cis(64, hd, 10000).float()
    def rot(x, p):  # fp32 rotation without output rounding
        c, s = table[p, :, 0], table[p, :, 1]
        x0, x1 = x.float()[..., :32], x.float()[..., 32:]
        return torch.cat([x0 * c - x1 * s, x1 * c + x0 * s], -1)
    d1 = (rot(q, 10) * rot(k, 7)).sum()
    d2 = (rot(q, 23) * rot(k, 20)).sum()
    assert abs(float(d1 - d2)) < 0.05 * float(q.float().norm() * k.float().norm())


# ---------------------------------------------------------------- norm / attention

def test_rms_norm_vs_library():
    x = torch.randn(4, 256, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    w = (torch.rand(256, generator=torch.Generator().manual_seed(7)) + 0.5).to(torch.bfloat16)
    ours = om.rms_norm(x, w, 1e-5)
    lib = F.rms_norm(x.float(), (256,), eps=1e-5).to(torch.bfloat16) * w
    assert float((ours.float() - lib.float()).abs().max()) <= 2 ** -6


def test_attention_vs_sdpa_gqa():
    H, NKV, T, hd = 8, 2, 37, 64
    g = torch.Generator().manual_seed(8)
    q = torch.randn(H, hd, generator=g).to(torch.bfloat16)
    kc = torch.randn(NKV, T, hd, generator=g).to(torch.bfloat16)
    vc = torch.randn(NKV, T, hd, generator=g).to(torch.bfloat16)
    valid = torch.ones(T, dtype=torch.bool)
    valid[30:] = False
    ours = om.attention(q, kc, vc, valid, 0.125).float().view(H, hd)
    k = kc.float().repeat_interleave(H // NKV, 0)
    v = vc.float().repeat_interleave(H // NKV, 0)
    lib = F.scaled_dot_product_attention(q.float().view(1, H, 1, hd), k.unsqueeze(0), v.unsqueeze(0),
                                         attn_mask=valid.view(1, 1, 1, T), scale=0.125)[0, :, 0]
    assert float((ours - lib).abs().max()) <= 2 ** -7
    # head h reads kv group h // 4: swapping groups changes the result
    swapped = om.attention(q, kc.flip(0), vc.flip(0), valid, 0.125).float().view(H, hd)
    assert float((swapped - lib).abs().max()) > 0.1


def test_attention_single_key_returns_v():
    """One visible key -> output = V of that key (reference bench/megakernel_decode_test.py:61-65)."""
    g = torch.Generator().manual_seed(9)
    q = torch.randn(4, 64, generator=g).to(torch.bfloat16)
    kc = torch.randn(2, 5, 64, generator=g).to(torch.bfloat16)
    vc = torch.randn(2, 5, 64, generator=g).to(torch.bfloat16)
    valid = torch.zeros(5, dtype=torch.bool)
    valid[0] = True
    out = om.attention(q, kc, vc, valid, 0.125).view(4, 64)
    assert torch.equal(out[0], vc[0, 0]) and torch.equal(out[3], vc[1, 0])


# ---------------------------------------------------------------- forward

def test_forward_chain_equals_sequential_steps():
    """verify-style M-token forward == M sequential decode steps (reference
    bench/verify_mega_test.py:43-59 invariant) on the oracle itself."""
    from flint_amd.synth import ModelArgs, synth_weights
    a = ModelArgs.from_name("tiny")
    sd = synth_weights(a, 2)
    o1, o2 = om.OracleModel(a, sd), om.OracleModel(a, sd)
    o1.setup_caches(32)
    o2.setup_caches(32)
    toks = torch.tensor([3, 99, 512, 7])
    l1, h1 = o1.forward(toks, 0)
    for i in range(4):
        l2, h2 = o2.forward(toks[i:i + 1], i)
        assert float((l1[i].float() - l2[0].float()).abs().max()) <= 2e-2
    assert torch.equal(o1.k_cache, o2.k_cache) or float((o1.k_cache.float() - o2.k_cache.float()).abs().max()) <= 0.05


def _tree(parent):
    """depth and ancestor-or-self mask of a tree given by parent indices (parent[0] = -1), as
    reference spec_tree.py:101-104 builds them."""
    m = len(parent)
    depth = torch.zeros(m, dtype=torch.int32)
    amask = torch.zeros(m, m, dtype=torch.uint8)
    for i in range(m):
        j = i
        while j >= 0:
            amask[i, j] = 1
            j = parent[j]
        depth[i] = int(amask[i].sum()) - 1
    return depth, amask


def _path(parent, i):
    p = []
    while i >= 0:
        p.append(i)
        i = parent[i]
    return p[::-1]


def test_forward_tree_rows_equal_chain_of_their_path():
    """The oracle's tree forward (depth / amask, reference verify_mega.cu:106-244 semantics and
    spec_tree.py:46-51): row i of an M-node tree verify equals the last row of a plain chain
    forward of the root -> i path at consecutive slots, for every node (RoPE at pos + depth, the
    same keys in the same order). A dropped ancestor in the mask or a depth off by one breaks it."""
    from flint_amd.synth import ModelArgs, synth_weights
    a = ModelArgs.from_name("tiny")
    sd = synth_weights(a, 3)
    pos = 9
    parent = [-1, 0, 0, 1, 1, 2, 3, 5, 3, 7]
    depth, amask = _tree(parent)
    g = torch.Generator().manual_seed(5)
    toks = torch.randint(0, a.vocab_size, (len(parent),), generator=g)
    kv = torch.randn(2, a.n_layer, a.n_local_heads, pos, 64, generator=g).to(torch.bfloat16)

    def model():
        o = om.OracleModel(a, sd)
        o.setup_caches(64)
        o.k_cache[:, :, :pos], o.v_cache[:, :, :pos] = kv[0], kv[1]
        return o
    o = model()
    tree, _ = o.forward(toks, pos, depth=depth, amask=amask)
    worst = 0.0
    for i in range(len(parent)):
        p = _path(parent, i)
        oc = model()
        chain, _ = oc.forward(toks[p], pos)
        d = float((tree[i].float() - chain[-1].float()).abs().max())
        worst = max(worst, d)
        assert d <= 2e-2, (i, p, d)
    # planted mistakes: node 6 (path 0-1-3-6) without its grandparent in the mask; node 9 with
    # every depth one too large
    bad = amask.clone()
    bad[6, 1] = 0
    o = model()
    wrong, _ = o.forward(toks, pos, depth=depth, amask=bad)
    oc = model()
    chain, _ = oc.forward(toks[_path(parent, 6)], pos)
    assert float((wrong[6].float() - chain[-1].float()).abs().max()) > 10 * max(worst, 1e-3)
    o = model()
    wrong, _ = o.forward(toks, pos, depth=depth + 1, amask=amask)
    oc = model()
    chain, _ = oc.forward(toks[_path(parent, 9)], pos)
    assert float((wrong[9].float() - chain[-1].float()).abs().max()) > 10 * max(worst, 1e-3)
