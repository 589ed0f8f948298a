"""CPU restatement of gpt-fast's sampling (reference engine/generate.py:36-55) and of the counter
RNG that drives the GPU sampler. Test infrastructure: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg use this module, as the checker of flint_amd's fl_sample.

Reference semantics (the logits are a bf16 tensor there, so every step is a bf16 tensor op: fp32
arithmetic rounded to bf16 at each op):

    logits = logits / max(temperature, 1e-5)                      generate.py:42
    v, _ = topk(logits, k); pivot = v[-1]                         :44-46
    logits = where(logits < pivot, -inf, logits)                  :47
    probs = softmax(logits)                                       :48
    q = empty_like(probs).exponential_(1)                         :37
    idx = argmax(probs / q)                                       :38

torch's exponential_ draws from its own Philox stream, which cannot be reproduced here; the GPU
sampler draws q from Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
as 1, 2, 3", SC 2011; the published Random123 known-answer vectors pin it) keyed by a caller seed,
with counter (vocab index, row, offset low, offset high), u = ((x0 >> 8) + 0.5) 2^-24 and
q = bf16(-log(u)) with the log in float64. Given the same q, the sample is a deterministic
function of the logits, and that function is what the GPU parity tests compare.

Pinned by: the Random123 known-answer vectors (Philox), the noise's moments and distance to
Exp(1), torch CPU's own bf16 ops on the same six lines (logits_to_probs_torch: within one bf16
ulp, nearly always identical), closed forms (top_k = 1 and constant noise give the argmax; ties
at the pivot stay) and the sample distribution (chi-square). The reference runs these ops on
CUDA, whose softmax and division may round the last fp32 bit differently from torch's CPU
kernels; that last-bit agreement is parity unpinned (no CUDA here), below the bf16 rounding that
follows except at rounding boundaries.
"""
import numpy as np
import torch

PHILOX_M0, PHILOX_M1 = 0xD2511F53, 0xCD9E8D57
PHILOX_W0, PHILOX_W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = 0xFFFFFFFF


def philox4x32_10(ctr, key):
    """Philox4x32 with 10 rounds. ctr: 4 uint32 arrays (broadcastable), key: 2 uint32 scalars.
    Returns 4 uint64 arrays holding uint32 values."""
    c = [np.asarray(x, dtype=np.uint64) & MASK32 for x in ctr]
    k0, k1 = int(key[0]) & MASK32, int(key[1]) & MASK32
    for r in range(10):
        if r:
            k0 = (k0 + PHILOX_W0) & MASK32
            k1 = (k1 + PHILOX_W1) & MASK32
        p0 = c[0] * np.uint64(PHILOX_M0)
        p1 = c[2] * np.uint64(PHILOX_M1)
        hi0, lo0 = p0 >> np.uint64(32), p0 & np.uint64(MASK32)
        hi1, lo1 = p1 >> np.uint64(32), p1 & np.uint64(MASK32)
        c = [hi1 ^ c[1] ^ np.uint64(k0), lo1, hi0 ^ c[3] ^ np.uint64(k1), lo0]
    return c


def uniform01(x0):
    """(0, 1) float64 from the top 24 bits of a uint32: ((x >> 8) + 0.5) * 2^-24 (exact)."""
    return ((np.asarray(x0, dtype=np.uint64) >> np.uint64(8)).astype(np.float64) + 0.5) * 2.0 ** -24


def bf16_round(a):
    """float32 -> nearest bf16 (ties to even), returned as float32."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    return torch.from_numpy(a.copy()).to(torch.bfloat16).float().numpy()


def exponential_noise(seed, offset, vocab, row=0):
    """q[i] = bf16(-log(u_i)) for i < vocab, u_i from Philox4x32-10 with key (seed lo, seed hi)
    and counter (i, row, offset lo, offset hi)."""
    i = np.arange(vocab, dtype=np.uint64)
    x = philox4x32_10([i, np.uint64(row), np.uint64(offset & MASK32), np.uint64((offset >> 32) & MASK32)],
                      (seed & MASK32, (seed >> 32) & MASK32))
    return bf16_round((-np.log(uniform01(x[0]))).astype(np.float32))


def logits_to_probs(logits, temperature=1.0, top_k=None):
    """generate.py:41-49 on a bf16 row (float32 array of bf16 values), step by step in float32
    with a bf16 rounding after each op; softmax divides exp(x - max) by the sum. Returns
    (probs bf16-valued float32, the scaled and masked logits)."""
    x = bf16_round(np.asarray(logits, dtype=np.float32) / np.float32(max(temperature, 1e-5)))
    if top_k is not None:
        k = min(int(top_k), x.size)
        pivot = np.sort(x)[::-1][k - 1]
        x = np.where(x < pivot, np.float32(-np.inf), x).astype(np.float32)
    mx = x.max()
    e = np.exp((x - mx).astype(np.float32)).astype(np.float32)
    s = np.float32(e.sum(dtype=np.float64))
    return bf16_round(e / s), x


def sample_with_noise(logits, q, temperature=1.0, top_k=None):
    """generate.py:36-38 with given noise q: argmax(bf16(probs / q)), the first index among ties.
    Returns (index, the bf16 ratios)."""
    probs, _ = logits_to_probs(logits, temperature, top_k)
    r = bf16_round(probs / np.asarray(q, dtype=np.float32))
    return int(np.argmax(r)), r


def logits_to_probs_torch(logits, temperature=1.0, top_k=None):
    """The same six lines as torch CPU bf16 ops (the reference's own code path, restated): a
    second restatement whose rounding differs from logits_to_probs only inside torch's softmax."""
    lg = torch.as_tensor(np.asarray(logits, dtype=np.float32)).to(torch.bfloat16)
    lg = lg / max(temperature, 1e-5)
    if top_k is not None:
        v, _ = torch.topk(lg, min(int(top_k), lg.size(-1)))
        pivot = v.select(-1, -1).unsqueeze(-1)
        lg = torch.where(lg < pivot, -float("Inf"), lg)
    return torch.nn.functional.softmax(lg, dim=-1)
