"""Model configuration and seeded synthetic weights.

ModelArgs mirrors reference engine/model.py:20-45 (field names and defaults of the fields this
engine uses). `CONFIGS` holds the synthetic 3B-class model the benchmark names plus small
shapes for tests. Weights are random (there is no checkpoint): linears N(0, 0.02) drawn in
fp32 then cast to bf16, norm weights |N(0,1)| + 0.5, tied embedding / LM head N(0, 0.02) bf16.
"""
from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass
class ModelArgs:
    block_size: int = 2048
    vocab_size: int = 32000
    n_layer: int = 32
    n_head: int = 32
    dim: int = 4096
    intermediate_size: Optional[int] = None
    n_local_heads: int = -1
    head_dim: int = 64
    rope_base: float = 10000
    norm_eps: float = 1e-5
    embedding_multiplier: float = 1.0
    attention_multiplier: Optional[float] = None
    residual_multiplier: float = 1.0
    logits_scaling: float = 1.0

    def __post_init__(self):
        if self.n_local_heads == -1:
            self.n_local_heads = self.n_head
        if self.intermediate_size is None:
            hidden = int(2 * 4 * self.dim / 3)
            self.intermediate_size = hidden + (-hidden) % 256
        self.head_dim = self.dim // self.n_head

    @property
    def attn_scale(self):
        return self.attention_multiplier if self.attention_multiplier is not None else self.head_dim ** -0.5

    @property
    def qkv_dim(self):
        return (self.n_head + 2 * self.n_local_heads) * self.head_dim

    @classmethod
    def from_name(cls, name):
        return cls(**CONFIGS[name])


CONFIGS = {
    # the benchmark's 40-layer 3B-class dense int4 model (and its one-layer parity variant)
    "flint-3b": dict(block_size=16384, n_layer=40, n_head=40, n_local_heads=8, dim=2560,
                     intermediate_size=8192, vocab_size=49152, rope_base=10000),
    "flint-3b-l1": dict(block_size=16384, n_layer=1, n_head=40, n_local_heads=8, dim=2560,
                        intermediate_size=8192, vocab_size=49152, rope_base=10000),
    # small shapes for fast parity tests (same head_dim 64 / group 128 constraints)
    "tiny": dict(block_size=1024, n_layer=2, n_head=8, n_local_heads=2, dim=512,
                 intermediate_size=1024, vocab_size=1024, rope_base=10000),
    "small": dict(block_size=2048, n_layer=4, n_head=20, n_local_heads=4, dim=1280,
                  intermediate_size=3072, vocab_size=4096, rope_base=10000),
    # the widest shape the decode kernel accepts (dim 3072, inter 8192): more weight chunks per
    # thread than the kernel's small chunk budget holds, so it runs the large-budget kernel
    "wide": dict(block_size=2048, n_layer=2, n_head=48, n_local_heads=8, dim=3072,
                 intermediate_size=8192, vocab_size=2048, rope_base=10000),
}


def synth_weights(args: ModelArgs, seed: int = 0, device="cpu"):
    """Seeded random bf16 weights in MODEL order (q heads | k heads | v heads for wqkv, rows in
    the HF/NEOX order). Keys: layers.{l}.{wqkv,wo,w1,w3,w2,attn_norm,ffn_norm}, norm, embed."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def lin(n, k):
        return (torch.randn(n, k, generator=g, device=device, dtype=torch.float32) * 0.02).to(torch.bfloat16)

    def normw(n):
        return (torch.randn(n, generator=g, device=device, dtype=torch.float32).abs() + 0.5).to(torch.bfloat16)

    D, F = args.dim, args.intermediate_size
    sd = {}
    for l in range(args.n_layer):
        p = f"layers.{l}."
        sd[p + "wqkv"] = lin(args.qkv_dim, D)
        sd[p + "wo"] = lin(D, D)
        sd[p + "w1"] = lin(F, D)
        sd[p + "w3"] = lin(F, D)
        sd[p + "w2"] = lin(D, F)
        sd[p + "attn_norm"] = normw(D)
        sd[p + "ffn_norm"] = normw(D)
    sd["norm"] = normw(D)
    sd["embed"] = lin(args.vocab_size, D)
    return sd


def freqs_cis_table(seq_len, n_elem, base, dtype=torch.bfloat16):
    """[seq_len, n_elem/2, 2] (cos, sin) table, computed on the CPU exactly as reference
    engine/model.py:245-254 precompute_freqs_cis defines it (fp32, then cast)."""
    freqs = 1.0 / (base ** (torch.arange(0, n_elem, 2)[: (n_elem // 2)].float() / n_elem))
    t = torch.arange(seq_len)
    ang = torch.outer(t, freqs)
    cis = torch.polar(torch.ones_like(ang), ang)
    return torch.stack([cis.real, cis.imag], dim=-1).to(dtype)
