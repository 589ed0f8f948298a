"""Greedy generation loop over the HIP decode kernel.

Mirrors reference engine/generate.py:57-81,137-206 (prefill / decode_one_token / decode_n_tokens /
generate) for greedy sampling and chat.py:71-96 (logits_at / pick / respond). Tokens stay on
the device between steps: step i reads the token step i-1 wrote, so the loop issues launches
back-to-back with no host synchronisation (gpt-fast's decode loop has none either). The prompt
is prefilled through the speculative-verify kernel, up to 32 tokens per launch.
"""
import torch


def prefill(model, x, input_pos, chunk=32):
    """Feed prompt tokens x (int32 device [T]) at positions input_pos[0]..; returns the greedy next
    token (int32 device [1]) after the last one (reference engine/generate.py:57-60, which runs
    the prompt through one forward). The prompt goes through the verify kernel `chunk` (<= 32)
    tokens per launch with a causal mask: each launch reads every weight once for the whole
    chunk and appends the chunk's K/V rows."""
    from . import _lib
    x = x.reshape(-1).to(device=model.device, dtype=torch.int32)
    p0 = int(input_pos.reshape(-1)[0]) if torch.is_tensor(input_pos) else int(input_pos)
    chunk = max(1, min(int(chunk), _lib.MAX_VERIFY))
    n = x.numel()
    out = torch.empty(1, dtype=torch.int32, device=model.device)
    if n == 0:
        return out
    cache = getattr(model, "_prefill_masks", None)
    if cache is None:
        cache = model._prefill_masks = {}
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        if m not in cache:
            cache[m] = (torch.arange(m, dtype=torch.int32, device=model.device),
                        torch.tril(torch.ones(m, m, dtype=torch.uint8, device=model.device)),
                        torch.empty(m, model.config.vocab_size, dtype=torch.float32, device=model.device),
                        torch.empty(m, model.config.dim, dtype=torch.bfloat16, device=model.device),
                        torch.empty(m, dtype=torch.int32, device=model.device))
        depth, amask, logits, feat, toks = cache[m]
        model.verify(x[s:s + m], p0 + s, depth=depth, amask=amask, logits=logits, feat=feat,
                     tokens_out=toks)
    out.copy_(toks[m - 1:m])
    return out


def sample(logits, temperature=1.0, top_k=None, seed=0, offset=0, noise=None, probs=False):
    """Sample one token per logit row on the GPU (reference engine/generate.py:36-55:
    logits_to_probs + multinomial_sample_one_no_sync). logits: fp32 device [V] or [rows, V]
    (bf16 values, as the decode and verify kernels write them). The exponential noise comes from
    Philox4x32-10 keyed by `seed` at counter (index, row, offset), or from `noise` (same shape as
    logits). Returns (tokens int32 device [rows], probs fp32 [rows, V] or None)."""
    from . import _lib
    lg = logits.float().contiguous()
    rows, vocab = (1, lg.numel()) if lg.dim() == 1 else (lg.shape[0], lg.shape[-1])
    if top_k is not None and int(top_k) < 1:
        raise ValueError("top_k must be >= 1")
    out = torch.empty(rows, dtype=torch.int32, device=lg.device)
    pr = torch.empty(rows, vocab, dtype=torch.float32, device=lg.device) if probs else None
    nz = None if noise is None else noise.float().contiguous()
    if nz is not None and nz.numel() != lg.numel():
        raise ValueError("noise must have the logits' shape")
    _lib.call("fl_sample", _lib.ptr(lg), rows, vocab, float(temperature), int(top_k or 0),
              int(seed) & (2 ** 64 - 1), int(offset) & (2 ** 64 - 1), _lib.ptr(nz), _lib.ptr(out),
              _lib.ptr(pr), _lib.stream_ptr())
    return out, pr


def logits_to_probs(logits, temperature=1.0, top_k=None):
    """Reference generate.py:41-49 on the GPU: probs fp32 device (bf16 values), logits' shape."""
    _, pr = sample(logits, temperature, top_k, probs=True)
    return pr.view(logits.shape)


def decode_one_token(model, x, input_pos, logits=None, temperature=None, top_k=None, seed=0):
    """(next_token int32 device [1], logits) for one token at input_pos: greedy, or sampled when
    temperature or top_k is given (reference generate.py:62-66, sample at :52-55), with the
    position as the noise counter."""
    pos = int(input_pos.reshape(-1)[0]) if torch.is_tensor(input_pos) else int(input_pos)
    if logits is None:
        logits = torch.empty(model.config.vocab_size, dtype=torch.float32, device=model.device)
    out = torch.empty(1, dtype=torch.int32, device=model.device)
    tok = x.reshape(-1)[:1].to(torch.int32)
    if temperature is not None or top_k is not None:  # sampled in the decode launch itself
        t = 1.0 if temperature is None else temperature
        model.decode_sample(tok, pos, t, top_k, seed=seed, offset=pos, token_out=out, logits=logits)
    else:
        model.decode_step(tok, pos, token_out=out, logits=logits)
    return out, logits


def decode_n_tokens(model, cur_token, input_pos, num_new_tokens, out=None):
    """Greedy-decode num_new_tokens tokens after cur_token (int32 device [1]) at input_pos.
    Returns int32 device [num_new_tokens]; no host synchronisation inside the loop."""
    pos = int(input_pos.reshape(-1)[0]) if torch.is_tensor(input_pos) else int(input_pos)
    buf = torch.empty(num_new_tokens + 1, dtype=torch.int32, device=model.device)
    buf[:1] = cur_token.reshape(-1)[:1]
    for i in range(num_new_tokens):
        model.decode_step(buf[i:i + 1], pos + i, token_out=buf[i + 1:i + 2])
    if out is not None:
        out.copy_(buf[1:])
        return out
    return buf[1:]


@torch.no_grad()
def generate(model, prompt, max_new_tokens, temperature=None, top_k=None, seed=0):
    """Generate: returns int32 device [T + max_new_tokens] = prompt + new tokens. Greedy (the
    argmax fused into the decode kernel) unless temperature or top_k is given; then each step
    samples in the decode launch itself (fl_decode_sample) with the step's position as the noise
    counter. Tokens stay on the device either way (no host synchronisation in the loop)."""
    prompt = prompt.reshape(-1).to(device=model.device, dtype=torch.int32)
    T = prompt.numel()
    model.setup_caches(1, T + max_new_tokens)
    seq = torch.empty(T + max_new_tokens, dtype=torch.int32, device=model.device)
    seq[:T] = prompt
    if T > 1:
        prefill(model, prompt[:-1], 0)
    sampled = temperature is not None or top_k is not None
    t = 1.0 if temperature is None else temperature
    # the last prompt token produces the first new token
    for i in range(max_new_tokens):
        p = T - 1 + i
        if sampled:
            model.decode_sample(seq[p:p + 1], p, t, top_k, seed=seed, offset=p, token_out=seq[p + 1:p + 2])
        else:
            model.decode_step(seq[p:p + 1], p, token_out=seq[p + 1:p + 2])
    return seq
