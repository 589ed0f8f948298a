"""The reference int4 decode path on the host CPU, used as bench.py's timed CPU baseline
(test infrastructure only; never part of the product).

gpt-fast runs every linear through aten::_weight_int4pack_mm on tinygemm-packed weights
(reference engine/quantize.py:359-373, 517-525). That CUDA op has no CPU kernel here; its CPU
counterparts aten::_convert_weight_to_int4pack_for_cpu / aten::_weight_int4pack_mm_for_cpu take
the same int32 [N, K] values and [K/128, N, 2] bf16 scales_and_zeros. The rest of the step is
oracle.model (norm, NEOX RoPE, fp32 attention, SwiGLU, tied bf16 LM head, greedy argmax).

torch's CPU int4 kernel does not round the dequantised weight twice as gpt-fast's Python
definition does (engine/quantize.py:152-154), so its outputs differ from oracle.model's linears by
up to one bf16 ulp on a large fraction of elements; tests/test_cpu_int4.py pins it at that level
and the whole step against oracle.model.
"""
import torch
import torch.nn.functional as F

from . import quant
from .model import attention, freqs_cis, rms_norm, rope_neox


class CpuInt4Linear:
    def __init__(self, w_bf16):
        q, s, z = quant.group_quantize(w_bf16)
        self.n = w_bf16.shape[0]
        self.w = torch.ops.aten._convert_weight_to_int4pack_for_cpu(q.cpu().contiguous(), 8)
        self.sz = quant.pack_scales_and_zeros(s, z).cpu()

    def __call__(self, x):
        return torch.ops.aten._weight_int4pack_mm_for_cpu(x, self.w, quant.GROUP, self.sz)


class CpuInt4Decoder:
    """Batch-1 greedy decode on the CPU with int4 linears. `sd` holds bf16 master weights (any
    device; quantisation runs where they live, the packed weights live on the CPU)."""

    def __init__(self, args, sd):
        self.args = a = args
        self.layers = []
        for l in range(a.n_layer):
            p = f"layers.{l}."
            self.layers.append(dict(
                wqkv=CpuInt4Linear(sd[p + "wqkv"]), wo=CpuInt4Linear(sd[p + "wo"]),
                w1=CpuInt4Linear(sd[p + "w1"]), w3=CpuInt4Linear(sd[p + "w3"]),
                w2=CpuInt4Linear(sd[p + "w2"]),
                attn_norm=sd[p + "attn_norm"].cpu(), ffn_norm=sd[p + "ffn_norm"].cpu()))
        self.norm = sd["norm"].cpu()
        self.embed = sd["embed"].cpu()
        self.table = freqs_cis(a.block_size, a.head_dim, a.rope_base)

    def setup_caches(self, max_seq, fill_upto=0, seed=0):
        a = self.args
        shape = (a.n_layer, a.n_local_heads, max_seq, a.head_dim)
        g = torch.Generator().manual_seed(seed)
        self.k = torch.zeros(shape, dtype=torch.bfloat16)
        self.v = torch.zeros(shape, dtype=torch.bfloat16)
        if fill_upto:
            self.k[:, :, :fill_upto] = torch.randn(*shape[:2], fill_upto, shape[3], generator=g).to(torch.bfloat16)
            self.v[:, :, :fill_upto] = torch.randn(*shape[:2], fill_upto, shape[3], generator=g).to(torch.bfloat16)

    def forward(self, tokens, pos):
        """Tokens (int [M]) at cache slots pos..pos+M-1, causal (engine/model.py:134-145 with
        input_pos = arange(pos, pos+M)): the M-row int4 linears run once for all tokens, the
        attention of token m covers slots [0, pos+m] (fp32 softmax, bf16 output). Returns the
        logits (bf16 [M, V])."""
        a = self.args
        hd = a.head_dim
        tokens = torch.as_tensor(tokens).reshape(-1).long()
        M = tokens.numel()
        x = self.embed[tokens] * a.embedding_multiplier
        rows = self.table[pos:pos + M]
        rep = a.n_head // a.n_local_heads
        T = pos + M
        mask = torch.ones(M, T, dtype=torch.bool).tril(diagonal=pos)
        for l, w in enumerate(self.layers):
            xn = rms_norm(x, w["attn_norm"], a.norm_eps)
            qkv = w["wqkv"](xn)
            q, k, v = qkv.split([a.n_head * hd, a.n_local_heads * hd, a.n_local_heads * hd], dim=-1)
            q = rope_neox(q.view(M, a.n_head, hd), rows)
            k = rope_neox(k.view(M, a.n_local_heads, hd), rows)
            self.k[l, :, pos:T] = k.transpose(0, 1)
            self.v[l, :, pos:T] = v.view(M, a.n_local_heads, hd).transpose(0, 1)
            if M == 1:
                y = attention(q[0], self.k[l, :, :T], self.v[l, :, :T], mask[0], a.attn_scale).view(1, -1)
            else:
                kk = self.k[l, :, :T].float().repeat_interleave(rep, dim=0)
                vv = self.v[l, :, :T].float().repeat_interleave(rep, dim=0)
                y = F.scaled_dot_product_attention(q.float().transpose(0, 1), kk, vv, attn_mask=mask,
                                                   scale=a.attn_scale)
                y = y.transpose(0, 1).reshape(M, -1).to(torch.bfloat16)
            h = x + w["wo"](y) * a.residual_multiplier
            hn = rms_norm(h, w["ffn_norm"], a.norm_eps)
            x = h + w["w2"](F.silu(w["w1"](hn)) * w["w3"](hn)) * a.residual_multiplier
        xn = rms_norm(x, self.norm, a.norm_eps)
        return F.linear(xn, self.embed) / a.logits_scaling

    def prefill(self, tokens, pos=0, chunk=128):
        """The prompt through forward `chunk` tokens at a time (reference engine/generate.py:57-60
        prefills in one forward); returns the greedy next token after the last one."""
        tokens = torch.as_tensor(tokens).reshape(-1)
        lg = None
        for s in range(0, tokens.numel(), chunk):
            lg = self.forward(tokens[s:s + chunk], pos + s)
        return int(torch.argmax(lg[-1]))

    def step_logits(self, token, pos):
        """Logits (bf16 [V]) of one decode step."""
        return self.forward(torch.tensor([int(token)]), pos)[0]

    def step(self, token, pos):
        """One greedy decode step (reference engine/generate.py:62-66 with argmax sampling)."""
        return int(torch.argmax(self.step_logits(token, pos)))
