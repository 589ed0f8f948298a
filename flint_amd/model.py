"""Engine host: packed int4 model on the GPU + gpt-fast-style API over the HIP decode kernel.

Mirrors the host side of reference engine/model.py:100-145 (Transformer.setup_caches /
forward(idx, input_pos, return_hidden)) and chat.py:23-52,71-77 (qpc/load_packed/logits_at):
weights are quantised once on the GPU into this library's layout, the KV cache is a caller-owned
bf16 tensor, and one decode step is ONE cooperative kernel launch (fl_decode_step).
"""
import torch

from . import _lib
from .quantize import quantize_int4, tile_int4
from .synth import ModelArgs, freqs_cis_table


def _find_multiple(n, k):
    return n if n % k == 0 else n + k - (n % k)


def qkv_storage_perm(args: ModelArgs):
    """Model row index for each packed QKV row: packed rows 2i / 2i+1 of a head hold the NEOX
    pair (i, i+32), so RoPE is local to a row pair in the kernel epilogue."""
    hd = args.head_dim
    nheads = args.n_head + 2 * args.n_local_heads
    i = torch.arange(hd // 2)
    within = torch.stack([i, i + hd // 2], dim=1).reshape(-1)  # [hd]
    return (torch.arange(nheads).unsqueeze(1) * hd + within.unsqueeze(0)).reshape(-1)


def gu_storage_rows(w1, w3):
    """Interleave gate (w1) and up (w3) rows: packed row 2i = w1[i], 2i+1 = w3[i]."""
    return torch.stack([w1, w3], dim=1).reshape(-1, w1.shape[1])


class PackedModel:
    """All layers' int4 weights (layer-stacked) + bf16 norms / embedding on one device."""

    def __init__(self, args: ModelArgs, sd, device="cuda"):
        self.args = args
        self.device = torch.device(device)
        L, D, F = args.n_layer, args.dim, args.intermediate_size
        nqkv = args.qkv_dim
        i32 = dict(dtype=torch.int32, device=self.device)
        self.wqkv_q = torch.empty(L, nqkv, D // 8, **i32)
        self.wqkv_sz = torch.empty(L, nqkv, D // 128, **i32)
        self.wo_q = torch.empty(L, D, D // 8, **i32)
        self.wo_sz = torch.empty(L, D, D // 128, **i32)
        self.wgu_q = torch.empty(L, 2 * F, D // 8, **i32)
        self.wgu_sz = torch.empty(L, 2 * F, D // 128, **i32)
        self.wd_q = torch.empty(L, D, F // 8, **i32)
        self.wd_sz = torch.empty(L, D, F // 128, **i32)
        perm = qkv_storage_perm(args).to(self.device)
        bf = dict(dtype=torch.bfloat16, device=self.device)
        for l in range(L):
            p = f"layers.{l}."
            dev = lambda t: t.to(**bf).contiguous()
            quantize_int4(dev(sd[p + "wqkv"]).index_select(0, perm).contiguous(),
                          self.wqkv_q[l], self.wqkv_sz[l])
            quantize_int4(dev(sd[p + "wo"]), self.wo_q[l], self.wo_sz[l])
            quantize_int4(gu_storage_rows(dev(sd[p + "w1"]), dev(sd[p + "w3"])).contiguous(),
                          self.wgu_q[l], self.wgu_sz[l])
            quantize_int4(dev(sd[p + "w2"]), self.wd_q[l], self.wd_sz[l])
        self.attn_norm = torch.stack([sd[f"layers.{l}.attn_norm"] for l in range(L)]).to(**bf).contiguous()
        self.ffn_norm = torch.stack([sd[f"layers.{l}.ffn_norm"] for l in range(L)]).to(**bf).contiguous()
        self.final_norm = sd["norm"].to(**bf).contiguous()
        self.embed = sd["embed"].to(**bf).contiguous()
        self.rope = freqs_cis_table(args.block_size, args.head_dim, args.rope_base).to(self.device).contiguous()
        self._tile()

    def _tile(self):
        """The four int4 matrices again in the tiled layout (fl_tile_int4), which the verify
        kernel's matrix-core tiles read; decode reads the row layout."""
        for name in ("wqkv", "wo", "wgu", "wd"):
            setattr(self, name + "_t", tile_int4(getattr(self, name + "_q")))

    @classmethod
    def from_tensors(cls, args: ModelArgs, t, device="cuda"):
        """A packed model from already-quantised tensors in this layout (flint_amd.checkpoint's
        packed file); shapes are checked against args."""
        self = object.__new__(cls)
        self.args = args
        self.device = torch.device(device)
        L, D, F, N = args.n_layer, args.dim, args.intermediate_size, args.qkv_dim
        want = {"wqkv_q": (L, N, D // 8), "wqkv_sz": (L, N, D // 128), "wo_q": (L, D, D // 8),
                "wo_sz": (L, D, D // 128), "wgu_q": (L, 2 * F, D // 8), "wgu_sz": (L, 2 * F, D // 128),
                "wd_q": (L, D, F // 8), "wd_sz": (L, D, F // 128), "attn_norm": (L, D), "ffn_norm": (L, D),
                "final_norm": (D,), "embed": (args.vocab_size, D)}
        for name, shp in want.items():
            x = t[name]
            if tuple(x.shape) != shp:
                raise ValueError(f"{name}: shape {tuple(x.shape)}, the model arguments need {shp}")
            dt = torch.int32 if name.endswith(("_q", "_sz")) else torch.bfloat16
            if x.dtype != dt:
                raise ValueError(f"{name}: dtype {x.dtype}, expected {dt}")
            setattr(self, name, x.to(self.device).contiguous())
        self.rope = freqs_cis_table(args.block_size, args.head_dim, args.rope_base).to(self.device).contiguous()
        self._tile()
        return self

    def nbytes_int4(self):
        """Bytes of one copy of the int4 weights with their scale/zero words (what one decode
        step reads; the tiled copies are verify's)."""
        return sum(t.numel() * 4 for t in (self.wqkv_q, self.wo_q, self.wgu_q, self.wd_q,
                                           self.wqkv_sz, self.wo_sz, self.wgu_sz, self.wd_sz))

    def c_weights(self):
        w = _lib.Weights()
        for name in ("wqkv_q", "wqkv_sz", "wo_q", "wo_sz", "wgu_q", "wgu_sz", "wd_q", "wd_sz",
                     "attn_norm", "ffn_norm", "final_norm", "embed", "rope",
                     "wqkv_t", "wo_t", "wgu_t", "wd_t"):
            setattr(w, name, getattr(self, name).data_ptr())
        w.rope_len = self.rope.shape[0]
        return w


class Transformer:
    """gpt-fast-style handle over the packed model and the HIP decode state."""

    def __init__(self, args: ModelArgs, packed: PackedModel):
        self.config = args
        self.packed = packed
        self.device = packed.device
        self.max_batch_size = -1
        self.max_seq_length = -1
        self._state = None
        self._cw = packed.c_weights()
        self.k_cache = self.v_cache = None

    @classmethod
    def from_weights(cls, args, sd, device="cuda"):
        return cls(args, PackedModel(args, sd, device))

    # reference engine/model.py:115-132
    def setup_caches(self, max_batch_size, max_seq_length):
        if max_batch_size != 1:
            raise ValueError("batch-1 decode engine: max_batch_size must be 1")
        if self.max_seq_length >= max_seq_length and self._state is not None:
            return
        self.close()
        a = self.config
        max_seq_length = _find_multiple(max_seq_length, 8)
        if max_seq_length > self.packed.rope.shape[0]:
            raise ValueError("max_seq_length exceeds block_size (rope table)")
        shape = (a.n_layer, a.n_local_heads, max_seq_length, a.head_dim)
        self.k_cache = torch.zeros(shape, dtype=torch.bfloat16, device=self.device)
        self.v_cache = torch.zeros(shape, dtype=torch.bfloat16, device=self.device)
        desc = _lib.ModelDesc(a.n_layer, a.dim, a.n_head, a.n_local_heads, a.intermediate_size,
                              a.vocab_size, a.norm_eps, a.embedding_multiplier, a.attn_scale,
                              a.residual_multiplier, a.logits_scaling)
        st = _lib.ctypes.c_void_p()
        _lib.call("fl_state_create", _lib.ctypes.byref(desc), max_seq_length,
                  _lib.ptr(self.k_cache), _lib.ptr(self.v_cache), _lib.ctypes.byref(st))
        self._state = st
        self.max_seq_length = max_seq_length
        self.max_batch_size = max_batch_size
        self._tok_out = torch.zeros(_lib.MAX_VERIFY, dtype=torch.int32, device=self.device)

    def close(self):
        if self._state is not None:
            _lib.call("fl_state_destroy", self._state)
            self._state = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def activations(self):
        """Diagnostics: the last launch's activations, copied out of the library's tagged exchange
        buffers (so no tensor keeps viewing library memory): h, attn [D] and act [F] as bf16 (each
        exchange word holds a bf16 value in its low 16 bits and a phase tag above), and qkv
        [(NH + 2 NKV) * 64] bf16 in model order (a word holds dims i and i + 32 of a head).
        Synchronises the current stream first."""
        torch.cuda.current_stream().synchronize()
        ptrs = [_lib.ctypes.c_void_p() for _ in range(4)]
        _lib.call("fl_state_buffers", self._state, *[_lib.ctypes.byref(p) for p in ptrs])
        a = self.config
        out = {}
        for k, p, n in (("h", ptrs[0], a.dim), ("attn", ptrs[2], a.dim), ("act", ptrs[3], a.intermediate_size)):
            w = _lib.device_view(p.value, n, torch.int32).clone()
            out[k] = (w & 0xFFFF).to(torch.int16).view(torch.bfloat16)
        w = _lib.device_view(ptrs[1].value, a.qkv_dim // 2, torch.int64).clone()
        lo = (w & 0xFFFF).to(torch.int16).view(torch.bfloat16).view(-1, 32)
        hi = ((w >> 16) & 0xFFFF).to(torch.int16).view(torch.bfloat16).view(-1, 32)
        out["qkv"] = torch.cat([lo, hi], dim=1).reshape(-1)
        return out

    def check(self):
        """Raise if a kernel recorded an error (synchronises)."""
        _lib.call("fl_state_check", self._state, _lib.stream_ptr())

    def reset_state(self):
        """Clear the decode state's error flag, counters and exchange buffers (not the KV cache)."""
        _lib.call("fl_state_reset", self._state, _lib.stream_ptr())

    def set_wait_limit(self, ticks=0):
        """Bound of the kernels' inter-workgroup waits in 100 MHz ticks (0: the default 2 s)."""
        _lib.call("fl_state_set_wait_limit", self._state, int(ticks))

    def force_timeout(self, on=True):
        """Tests: later launches start with a wait that is never satisfied (the timeout path)."""
        _lib.call("fl_state_force_timeout", self._state, 1 if on else 0)

    def decode_step(self, token, pos, token_out=None, logits=None, feat=None):
        """One decode step: token (int32 device tensor, 1 element) at position pos. Writes the greedy
        argmax to token_out (int32 device, 1 element; default: an internal buffer) and returns it."""
        if self._state is None:
            raise RuntimeError("call setup_caches first")
        if token_out is None:
            token_out = self._tok_out[:1]
        for t, dt, nm in ((token, torch.int32, "token"), (token_out, torch.int32, "token_out"),
                          (logits, torch.float32, "logits"), (feat, torch.bfloat16, "feat")):
            if t is not None and (not t.is_cuda or t.dtype != dt):
                raise ValueError(f"{nm} must be a {dt} device tensor")
        _lib.call("fl_decode_step", _lib.ctypes.byref(self._cw), self._state, _lib.ptr(token), int(pos),
                  _lib.ptr(token_out), _lib.ptr(logits), _lib.ptr(feat), _lib.stream_ptr())
        return token_out

    def decode_sample(self, token, pos, temperature=1.0, top_k=None, seed=0, offset=None,
                      token_out=None, logits=None, feat=None):
        """One decode step whose token is sampled in the same launch (temperature / top-k, reference
        engine/generate.py:38-55): Philox noise keyed by seed at counter offset (default: pos).
        Returns token_out (int32 device [1])."""
        if self._state is None:
            raise RuntimeError("call setup_caches first")
        if token_out is None:
            token_out = self._tok_out[:1]
        for t, dt, nm in ((token, torch.int32, "token"), (token_out, torch.int32, "token_out"),
                          (logits, torch.float32, "logits"), (feat, torch.bfloat16, "feat")):
            if t is not None and (not t.is_cuda or t.dtype != dt):
                raise ValueError(f"{nm} must be a {dt} device tensor")
        if top_k is not None and int(top_k) < 1:
            raise ValueError("top_k must be >= 1")
        off = int(pos) if offset is None else int(offset)
        _lib.call("fl_decode_sample", _lib.ctypes.byref(self._cw), self._state, _lib.ptr(token), int(pos),
                  float(temperature), int(top_k or 0), int(seed) & (2 ** 64 - 1), off & (2 ** 64 - 1),
                  _lib.ptr(token_out), _lib.ptr(logits), _lib.ptr(feat), _lib.stream_ptr())
        return token_out

    def decode_hidden(self, h, pos, token_out=None, logits=None, feat=None):
        """One decode step from a hidden state (reference decode_mega_launch's h argument): h (bf16
        [D] device tensor) is the layer-0 input and holds the final residual afterwards (in place).
        Optional outputs as decode_step; returns token_out (None if not given)."""
        if self._state is None:
            raise RuntimeError("call setup_caches first")
        for t, dt, nm in ((h, torch.bfloat16, "h"), (token_out, torch.int32, "token_out"),
                          (logits, torch.float32, "logits"), (feat, torch.bfloat16, "feat")):
            if t is not None and (not t.is_cuda or t.dtype != dt):
                raise ValueError(f"{nm} must be a {dt} device tensor")
        if h.numel() != self.config.dim or not h.is_contiguous():
            raise ValueError(f"h must be a contiguous [{self.config.dim}] tensor")
        _lib.call("fl_decode_hidden", _lib.ctypes.byref(self._cw), self._state, _lib.ptr(h), int(pos),
                  _lib.ptr(token_out), _lib.ptr(logits), _lib.ptr(feat), _lib.stream_ptr())
        return token_out

    def verify(self, tokens, pos, depth=None, amask=None, logits=None, feat=None, tokens_out=None):
        """Speculative verify of M tokens at cache slots pos..pos+M-1 (reference verify_mega_launch).
        depth (int32 [M], default arange) gives RoPE positions pos+depth; amask (uint8 [M,M], default
        causal) the tree mask. Returns (argmax tokens [M], logits [M,V] fp32, feat [M,D] bf16);
        logits=False / feat=False skip writing that output (None is returned in its place)."""
        if self._state is None:
            raise RuntimeError("call setup_caches first")
        m = tokens.numel()
        dev = self.device
        if depth is None:
            depth = torch.arange(m, dtype=torch.int32, device=dev)
        if amask is None:
            amask = torch.tril(torch.ones(m, m, dtype=torch.uint8, device=dev))
        if logits is None:
            logits = torch.empty(m, self.config.vocab_size, dtype=torch.float32, device=dev)
        elif logits is False:
            logits = None
        if feat is None:
            feat = torch.empty(m, self.config.dim, dtype=torch.bfloat16, device=dev)
        elif feat is False:
            feat = None
        if tokens_out is None:
            tokens_out = torch.empty(m, dtype=torch.int32, device=dev)
        _lib.call("fl_verify", _lib.ctypes.byref(self._cw), self._state, _lib.ptr(tokens.int().contiguous()),
                  m, _lib.ptr(depth.int().contiguous()), _lib.ptr(amask.to(torch.uint8).contiguous()), int(pos),
                  _lib.ptr(tokens_out), _lib.ptr(logits), _lib.ptr(feat), _lib.stream_ptr())
        return tokens_out, logits, feat

    def kv_move(self, src, dst):
        """Move the K/V rows of cache slots src[i] to dst[i] in every layer (host int lists, at most
        32): the KV compaction after a tree verify (reference spec_tree.py:124-127). All rows are
        read before any is written."""
        if self._state is None:
            raise RuntimeError("call setup_caches first")
        n = len(src)
        if n != len(dst):
            raise ValueError("src and dst must have the same length")
        arr = _lib.ctypes.c_int32 * max(n, 1)
        _lib.call("fl_kv_move", self._state, arr(*src), arr(*dst), n, _lib.stream_ptr())

    # reference engine/model.py:134-145 (decode: one token per call)
    def forward(self, idx, input_pos, return_hidden=False):
        idx = idx.reshape(-1).to(device=self.device, dtype=torch.int32)
        pos = int(input_pos.reshape(-1)[0]) if torch.is_tensor(input_pos) else int(input_pos)
        n = idx.numel()
        logits = torch.empty(n, self.config.vocab_size, dtype=torch.float32, device=self.device)
        feat = torch.empty(n, self.config.dim, dtype=torch.bfloat16, device=self.device)
        for i in range(n):
            self.decode_step(idx[i:i + 1], pos + i, logits=logits[i], feat=feat[i])
        logits = logits.view(1, n, -1)
        return (logits, feat.view(1, n, -1)) if return_hidden else logits
