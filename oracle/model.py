"""gpt-fast forward pass on dequantised int4 weights, restated on the CPU (test infrastructure only).

Follows reference engine/model.py:134-242 op by op in bf16 so every rounding point matches:
  x      = bf16(embed[idx] * emb_mult)                                   (model.py:138)
  h      = bf16(x + bf16(attn(norm(x)) * rm))                             (model.py:162)
  out    = bf16(h + bf16(ffn(norm(h)) * rm))                              (model.py:163)
  norm   = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)                     (model.py:237-242)
  linear = bf16(sum_k x_k * dq_nk), fp32 accumulation                     (quantize.py:517-525)
  ffn    = w2(bf16(bf16(silu(w1 x)) * w3 x))                              (model.py:227-228)
  logits = bf16(bf16(norm(x) . E^T) / logits_scaling), tied E            (model.py:143-144)
RoPE is the NEOX half-split form (pairs i, i+32) with gpt-fast's bf16 cos/sin table
(model.py:245-269 applied to permuted rows, convert_hf_checkpoint.py:75-81). Attention is
softmax(q.k^T * scale) v in fp32 with one bf16 rounding of the output (the reduced-precision math
SDPA path upcasts to fp32), GQA head h reading kv head h // (n_head / n_kv)  (model.py:210-212).
The KV cache has the engine's layout [NL, NKV, S, 64].
"""
import torch
import torch.nn.functional as F

from . import quant


def _bf(t):
    return t.to(torch.bfloat16)


def freqs_cis(seq_len, n_elem, base):
    """bf16 [seq_len, n_elem/2, 2] cos/sin table. Restates reference engine/model.py:245-254."""
    inv = 1.0 / (base ** (torch.arange(0, n_elem, 2)[: (n_elem // 2)].float() / n_elem))
    ang = torch.outer(torch.arange(seq_len), inv)
    cis = torch.polar(torch.ones_like(ang), ang)
    return torch.stack([cis.real, cis.imag], dim=-1).to(torch.bfloat16)


def rms_norm(x, w, eps):
    """Restates reference engine/model.py:231-242 RMSNorm (x bf16 [..., D], w bf16 [D])."""
    xf = x.float()
    n = (xf * torch.rsqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + eps)).to(x.dtype)
    return n * w


def rope_neox(x, table_rows):
    """NEOX half-split RoPE of bf16 x [..., M, H, 64] with table rows [M, 32, 2] (bf16), computed in
    fp32 with the products rounded separately, result bf16 (reference engine/model.py:257-269
    on the pair (i, i+32))."""
    half = x.shape[-1] // 2
    xf = x.float()
    x0, x1 = xf[..., :half], xf[..., half:]
    c = table_rows[..., 0].float().unsqueeze(-2)   # [M, 1, 32]
    s = table_rows[..., 1].float().unsqueeze(-2)
    o0 = x0 * c - x1 * s
    o1 = x1 * c + x0 * s
    return torch.cat([o0, o1], dim=-1).to(x.dtype)


def rope_interleaved(x, table_rows):
    """gpt-fast's interleaved RoPE (pairs 2i, 2i+1), reference engine/model.py:257-269; used only
    to pin rope_neox through the permutation identity."""
    xs = x.float().reshape(*x.shape[:-1], -1, 2)
    c = table_rows[..., 0].float().unsqueeze(-2)
    s = table_rows[..., 1].float().unsqueeze(-2)
    o = torch.stack([xs[..., 0] * c - xs[..., 1] * s, xs[..., 1] * c + xs[..., 0] * s], dim=-1)
    return o.flatten(-2).to(x.dtype)


def hf_to_interleaved_perm(n_heads, head_dim):
    """Row permutation HF(NEOX) -> gpt-fast interleaved order
    (reference engine/scripts/convert_hf_checkpoint.py:75-81 permute)."""
    i = torch.arange(head_dim // 2)
    within = torch.stack([i, i + head_dim // 2], dim=1).reshape(-1)
    return (torch.arange(n_heads).unsqueeze(1) * head_dim + within.unsqueeze(0)).reshape(-1)


def linear_g128(x, w):
    """x . w^T with fp32 partial sums per 128-column group added in group order (bf16 result): a
    second valid fp32 summation order of the reference linear (engine/quantize.py:517-525 fixes
    the operands and the bf16 rounding of the result, not the order of the fp32 sum). Used to
    measure the order-noise floor of the reference semantics on the inputs of a test."""
    K = x.shape[-1]
    acc = None
    for b in range(0, K, 128):
        part = x[..., b:b + 128].float() @ w[:, b:b + 128].float().T
        acc = part if acc is None else acc + part
    return acc.to(x.dtype)


LOG2E = 1.4426950408889634


def softmax_exp2(s):
    """fp32 softmax with exp written as exp2(x * log2 e) (another valid fp32 implementation of the
    reference softmax: the reference fixes the operation, not the last ulp of its exp)."""
    p = torch.exp2((s - s.amax(dim=-1, keepdim=True)) * LOG2E)
    return p / p.sum(dim=-1, keepdim=True)


def silu_exp2(x):
    """bf16 SiLU computed in fp32 as x * 1 / (1 + exp2(-x log2 e)) (another valid implementation
    of torch's F.silu on a bf16 tensor: same operation, fp32 inside, one bf16 rounding)."""
    xf = x.float()
    return (xf * (1.0 / (1.0 + torch.exp2(-xf * LOG2E)))).to(x.dtype)


# Named implementations of the reference semantics: (linear, softmax, silu). Every one fixes the
# same operations and bf16 rounding points; they differ in fp32 summation order and in the last
# ulps of exp, which is the freedom any implementation (the reference's own GPU path included) has.
IMPLS = {
    "torch": (F.linear, torch.softmax, F.silu),
    "g128": (linear_g128, torch.softmax, F.silu),
    "exp2": (F.linear, softmax_exp2, silu_exp2),
    "g128+exp2": (linear_g128, softmax_exp2, silu_exp2),
}
LINEAR_ORDERS = {k: v[0] for k, v in IMPLS.items()}


def attention(q, kc, vc, valid, scale, softmax=torch.softmax):
    """q bf16 [H, 64]; kc, vc bf16 [NKV, T, 64]; valid bool [T]. fp32 softmax attention, bf16 out [H*64]."""
    H, NKV = q.shape[0], kc.shape[0]
    rep = H // NKV
    k = kc[:, valid].float().repeat_interleave(rep, dim=0)   # [H, T', 64]
    v = vc[:, valid].float().repeat_interleave(rep, dim=0)
    s = torch.einsum("hd,htd->ht", q.float(), k) * scale
    p = softmax(s, dim=-1) if softmax is torch.softmax else softmax(s)
    o = torch.einsum("ht,htd->hd", p, v)
    return o.to(torch.bfloat16).reshape(-1)


class OracleModel:
    """CPU restatement of the reference int4 model. sd: bf16 master weights in model order
    (flint_amd.synth.synth_weights keys). Linears are quantised/dequantised by oracle.quant."""

    def __init__(self, args, sd, quantize=True):
        self.args = a = args
        self.L = a.n_layer
        dq = quant.dq_linear_weight if quantize else (lambda w: w)
        self.w = []
        for l in range(a.n_layer):
            p = f"layers.{l}."
            self.w.append(dict(
                wqkv=dq(sd[p + "wqkv"].cpu()), wo=dq(sd[p + "wo"].cpu()),
                w1=dq(sd[p + "w1"].cpu()), w3=dq(sd[p + "w3"].cpu()), w2=dq(sd[p + "w2"].cpu()),
                attn_norm=sd[p + "attn_norm"].cpu(), ffn_norm=sd[p + "ffn_norm"].cpu()))
        self.norm = sd["norm"].cpu()
        self.embed = sd["embed"].cpu()
        self.table = freqs_cis(a.block_size, a.head_dim, a.rope_base)
        self.k_cache = self.v_cache = None
        self.linear, self.softmax, self.silu = IMPLS["torch"]
        self.last_residual = None
        # trace: when a list, forward() appends per layer a dict of that layer's input and
        # intermediate values (q, k, v after RoPE, attention output, SwiGLU output, output)
        self.trace = None
        self._rec = None

    def set_order(self, name):
        """Implementation of the reference semantics (IMPLS): "torch" (the default), "g128",
        "exp2" or "g128+exp2". All are the reference semantics; their differences are the
        noise floor any implementation has."""
        self.linear, self.softmax, self.silu = IMPLS[name]

    def setup_caches(self, max_seq):
        a = self.args
        shape = (a.n_layer, a.n_local_heads, max_seq, a.head_dim)
        self.k_cache = torch.zeros(shape, dtype=torch.bfloat16)
        self.v_cache = torch.zeros(shape, dtype=torch.bfloat16)
        self.max_seq = max_seq

    def layer_attention(self, l, x, pos, depth=None, amask=None):
        """Attention block of layer l for the M tokens x (bf16 [M, D]) at cache slots pos..pos+M-1.
        RoPE position of token m is pos + depth[m]; token m attends to slots [0, pos) and to the slots
        pos + j with amask[m, j] (default: causal chain)."""
        a, w = self.args, self.w[l]
        M, hd = x.shape[0], a.head_dim
        depth = torch.arange(M) if depth is None else depth
        amask = torch.tril(torch.ones(M, M, dtype=torch.bool)) if amask is None else amask.bool()
        xn = rms_norm(x, w["attn_norm"], a.norm_eps)
        qkv = self.linear(xn, w["wqkv"])
        q, k, v = qkv.split([a.n_head * hd, a.n_local_heads * hd, a.n_local_heads * hd], dim=-1)
        rows = self.table[pos + depth]                        # [M, 32, 2]
        q = rope_neox(q.view(M, a.n_head, hd), rows)
        k = rope_neox(k.view(M, a.n_local_heads, hd), rows)
        v = v.view(M, a.n_local_heads, hd)
        self.k_cache[l, :, pos:pos + M] = k.transpose(0, 1)
        self.v_cache[l, :, pos:pos + M] = v.transpose(0, 1)
        T = pos + M
        ys = []
        for m in range(M):
            valid = torch.zeros(T, dtype=torch.bool)
            valid[:pos] = True
            valid[pos:pos + M] = amask[m]
            ys.append(attention(q[m], self.k_cache[l, :, :T], self.v_cache[l, :, :T], valid, a.attn_scale,
                                self.softmax))
        y = torch.stack(ys)
        if self._rec is not None:
            self._rec.update(q=q.reshape(M, -1), k=k.reshape(M, -1), v=v.reshape(M, -1), attn=y)
        return self.linear(y, w["wo"])

    def layer(self, l, x, pos, depth=None, amask=None):
        """Decoder block l on the M tokens x (bf16 [M, D]) at cache slots pos..pos+M-1 (reference
        engine/model.py:160-164): h = x + attn(norm(x)) * rm; out = h + ffn(norm(h)) * rm."""
        a, w, lin = self.args, self.w[l], self.linear
        self._rec = {"x": x} if self.trace is not None else None
        h1 = x + self.layer_attention(l, x, pos, depth, amask) * a.residual_multiplier
        hn = rms_norm(h1, w["ffn_norm"], a.norm_eps)
        act = self.silu(lin(hn, w["w1"])) * lin(hn, w["w3"])
        out = h1 + lin(act, w["w2"]) * a.residual_multiplier
        if self._rec is not None:
            self._rec.update(act=act, out=out)
            self.trace.append(self._rec)
            self._rec = None
        return out

    def forward(self, idx, pos, depth=None, amask=None, h=None):
        """idx int [M] at cache slots pos..pos+M-1 -> (logits bf16 [M, V], post-norm hidden bf16 [M, D]).
        With h (bf16 [M, D]) the layer-0 input is h itself instead of the scaled embedding (the
        reference megakernel's h argument, kernels/megakernel_decode.cu:204-208); idx is then
        ignored. The final residual (before the final norm) is kept in self.last_residual."""
        a = self.args
        lin = self.linear
        x = h.to(torch.bfloat16) if h is not None else self.embed[idx.long()] * a.embedding_multiplier
        for l in range(self.L):
            x = self.layer(l, x, pos, depth, amask)
        self.last_residual = x
        xn = rms_norm(x, self.norm, a.norm_eps)
        logits = lin(xn, self.embed) / a.logits_scaling
        return logits, xn

    def decode_greedy(self, token, pos, steps):
        """Greedy decode `steps` tokens after `token` at `pos` (reference engine/generate.py:68-81 with
        argmax sampling). Returns (tokens [steps], logits list)."""
        toks, logs = [], []
        cur = int(token)
        for i in range(steps):
            lg, _ = self.forward(torch.tensor([cur]), pos + i)
            cur = int(torch.argmax(lg[0]))
            toks.append(cur)
            logs.append(lg[0])
        return torch.tensor(toks, dtype=torch.int32), logs
