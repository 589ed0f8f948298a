/*
 * flint_amd.h — C ABI of the MI355X (gfx950) batch-1 int4 decode engine.
 *
 * Every entry point takes plain device pointers and sizes, is stream-ordered on the
 * hipStream_t passed as `stream` (NULL = the legacy default stream), allocates nothing
 * on the decode/verify hot path, and returns an int status: FL_OK (0) or a negative
 * FL_E* code. Nothing here is thread-safe for a shared fl_state.
 *
 * Weight layout (owned by this library; produced by fl_quantize_int4):
 *   q  : uint32 [N, K/8]    row-major; word j of a row holds elements 8j..8j+7, element
 *                           8j+2i at bits 4i and element 8j+2i+1 at bits 16+4i (i = 0..3)
 *   sz : uint32 [N, K/128]  per (row, 128-group): bits 0..15 = scale (bf16),
 *                           bits 16..31 = zero (bf16)
 * Values follow gpt-fast's asymmetric group quantisation
 *   (reference engine/quantize.py:58-76 get_group_qparams, :102-128 quantise),
 * and dequantise to  bf16( bf16((q-8)*scale) + zero )  (reference engine/quantize.py:138-155).
 *
 * bf16 values are passed as uint16_t bit patterns.
 */
#ifndef FLINT_AMD_H
#define FLINT_AMD_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FL_OK = 0,
  FL_E_ARG = -1,        /* null pointer / bad size / unsupported shape                         */
  FL_E_POS = -2,        /* pos (+ M) beyond the state's max_seq or the rope table              */
  FL_E_M = -3,          /* verify width M outside 1..FL_MAX_VERIFY                             */
  FL_E_LAUNCH = -4,     /* HIP launch failed (e.g. a cooperative grid cannot be co-resident)   */
  FL_E_HIP = -5,        /* other HIP runtime error (allocation, copy)                          */
  FL_E_TIMEOUT = -6     /* an inter-workgroup wait hit its 2 s limit in an earlier launch (e.g.
                           a workgroup was not resident because other work held its CU)        */
};

#define FL_MAX_VERIFY 32
#define FL_HEAD_DIM 64
#define FL_GROUP 128

/* Model shape and scalar multipliers. Mirrors reference engine/model.py:20-45 ModelArgs
 * (head_dim fixed at 64, group size fixed at 128). */
typedef struct fl_model_desc {
  int32_t n_layer, dim, n_head, n_kv_head, inter, vocab;
  float norm_eps, emb_mult, attn_scale, resid_mult, logits_scaling;
} fl_model_desc;

/* Device pointers to one model's packed weights (caller-owned). Layer-stacked.
 * QKV rows are stored NEOX-pair-interleaved: packed row 2i / 2i+1 of head h holds
 *   model row h*64 + i / h*64 + i + 32  (i < 32), heads ordered [q heads | k heads | v heads].
 * Gate/up rows are interleaved: packed row 2i = w1 row i (gate), 2i+1 = w3 row i (up). */
typedef struct fl_weights {
  const uint32_t *wqkv_q, *wqkv_sz;   /* [NL, (NH+2*NKV)*64, D/8], [.., D/128]  */
  const uint32_t *wo_q, *wo_sz;       /* [NL, D, D/8], [NL, D, D/128]           */
  const uint32_t *wgu_q, *wgu_sz;     /* [NL, 2F, D/8], [NL, 2F, D/128]         */
  const uint32_t *wd_q, *wd_sz;       /* [NL, D, F/8], [NL, D, F/128]           */
  const uint16_t *attn_norm;          /* [NL, D] bf16                            */
  const uint16_t *ffn_norm;           /* [NL, D] bf16                            */
  const uint16_t *final_norm;         /* [D] bf16                                */
  const uint16_t *embed;              /* [V, D] bf16, tied LM head               */
  const uint16_t *rope;               /* [rope_len, 32, 2] bf16 (cos, sin)       */
  int32_t rope_len;
  /* The same four int4 matrices in the tiled layout (fl_tile_int4 of each layer-stacked matrix,
   * same sizes as wqkv_q .. wd_q): fl_verify's matrix-core tiles read these, the decode entry
   * points the row layout above. Required by fl_verify only. */
  const uint32_t *wqkv_t, *wo_t, *wgu_t, *wd_t;
} fl_weights;

typedef struct fl_state fl_state;

/* Library/device information. */
int fl_version(void);
int fl_device_info(int32_t* num_cu, int32_t* decode_grid);

/* ---- quantisation / dequantisation / standalone GEMV --------------------------------- */

/* Group-wise int4 quantisation of a bf16 [N,K] matrix (K % 128 == 0).
 * Replaces reference engine/quantize.py:131-135 group_quantize_tensor (+ :359-364 prepare_...). */
int fl_quantize_int4(const uint16_t* w, uint32_t* q, uint32_t* sz,
                     int32_t n, int32_t k, void* stream);

/* Bit-exact dequantisation to bf16 [N,K] on the vector ALUs, the device routine of
 * fl_gemm_int4.
 * Replaces reference engine/quantize.py:138-162 group_dequantize_tensor(_from_qparams). */
int fl_dequant_int4(const uint32_t* q, const uint32_t* sz, uint16_t* out,
                    int32_t n, int32_t k, void* stream);
/* The same bits through the matrix-core form of the dequantisation that the decode kernel's
 * GEMVs and fl_gemv_int4 run (both rounding steps as 4x4x4 MFMAs, lane by lane). Replaces reference
 * engine/quantize.py:138-162 as fl_dequant_int4 does; kept apart so that each form is checked. */
int fl_dequant_int4_mx(const uint32_t* q, const uint32_t* sz, uint16_t* out,
                       int32_t n, int32_t k, void* stream);

/* y[N] = bf16( sum_k x[k] * dq[n,k] ), fp32 accumulation. M=1 int4 GEMV.
 * Replaces reference engine/quantize.py:517-525 WeightOnlyInt4Linear.forward ->
 * aten::_weight_int4pack_mm (:370) at M=1, and kernels/int4_gemv.cu:383-424 int4_gemv_v. */
int fl_gemv_int4(const uint32_t* q, const uint32_t* sz, const uint16_t* x, uint16_t* y,
                 int32_t n, int32_t k, void* stream);

/* Y[M,N] = bf16( X[M,K] . dq[N,K]^T ), M <= FL_MAX_VERIFY (32), weight read once for all M rows.
 * Replaces reference kernels/int4_gemv_mk.cu:11-57 gemv_mk<M> and kernels/int4_gemm_tc.cu:12-70. */
int fl_gemm_int4(const uint32_t* q, const uint32_t* sz, const uint16_t* x, uint16_t* y,
                 int32_t m, int32_t n, int32_t k, void* stream);

/* ---- tiled layout: the exact dequantisation on the matrix cores ------------------------- */

/* The same int4 values in the tiled layout the matrix-core kernels read (N % 16 == 0): per block
 * of 16 rows and 128-column group, 1 KB; 16 bytes per lane l of a wave, with p = (l / 4) % 4 and
 * c = 4 (l / 16) + l % 4: words 0 / 1 hold rows 4p, 4p+1 at columns c + 16t (t = 0..3 / 4..7: row
 * 4p at bits 4(t%4), row 4p+1 at 16 + 4(t%4)), words 2 / 3 the same for rows 4p+2, 4p+3.
 * qt: uint32 [N/16, K/128, 64, 4]; sz is unchanged.
 * No counterpart in the reference (its tinygemm tile layout, quantize.py:359-364, serves the
 * same purpose for its CUDA kernel). */
int fl_tile_int4(const uint32_t* q, uint32_t* qt, int32_t n, int32_t k, void* stream);
/* Bit-exact dequantisation of a tiled matrix to bf16 [N,K] (row order) through the GEMV's own
 * matrix-core steps. Replaces reference engine/quantize.py:138-162 for the tiled layout. */
int fl_dequant_int4_tiled(const uint32_t* qt, const uint32_t* sz, uint16_t* out, int32_t n, int32_t k,
                          void* stream);
/* y[N] = bf16( sum_k x[k] * dq[n,k] ), M = 1, from the tiled layout: both exact dequantisation
 * steps and the dot on the matrix cores. Replaces reference engine/quantize.py:517-525
 * WeightOnlyInt4Linear.forward at M = 1 and kernels/int4_gemv.cu:383-424 int4_gemv_v. */
int fl_gemv_int4_tiled(const uint32_t* qt, const uint32_t* sz, const uint16_t* x, uint16_t* y, int32_t n,
                       int32_t k, void* stream);

/* ---- decode state --------------------------------------------------------------------- */

/* Binds a caller-owned bf16 KV cache (k_cache, v_cache: [NL, NKV, max_seq, 64] each, device)
 * and allocates all decode/verify scratch once (hipMalloc here, never on the hot path).
 * Replaces the per-call torch::empty scratch of reference kernels/megakernel_decode.cu:212-223;
 * the caller-owned cache mirrors reference chat.py:68-69 / engine/model.py:82-98 KVCache. */
int fl_state_create(const fl_model_desc* desc, int32_t max_seq, uint16_t* k_cache,
                    uint16_t* v_cache, fl_state** out);
int fl_state_destroy(fl_state* st);
/* Zero all scratch counters and exchange buffers (not the KV cache). The exchange buffers are
 * also zeroed every few hundred launches by the launches themselves (a kernel on the launch's
 * stream), before their 16-bit tags could come round to a value an old word still carries. */
int fl_state_reset(fl_state* st, void* stream);
/* Diagnostics, no counterpart in the reference: when buf (device, uint64 [grid * slots_per_wg])
 * is non-NULL, every later decode launch writes per-workgroup timestamps of the 100 MHz
 * real-time clock: slot 0 at kernel start, then 12 per layer (for each of the 5 phases when its
 * inputs have arrived and when its epilogue is done, plus the attention phase's inputs / loop /
 * merge), then the final norm's input arrival and the end of the LM head. NULL disables.
 * *grid receives the number of workgroups. */
int fl_state_profile(fl_state* st, uint64_t* buf, int32_t slots_per_wg, int32_t* grid);
/* Diagnostics, no counterpart in the reference: device pointers of the last launch's tagged
 * exchange buffers (token row 0): residual h [D], attention output [D] and SwiGLU output [F] as
 * uint32 words (bf16 bits | phase tag << 16), and this step's q/k/v as uint64 words [(NH+2*NKV)*32]
 * (bf16 bits of dim i | bf16 bits of dim i+32 << 16 | tag << 32; word hh*32+i, heads [q|k|v]). */
int fl_state_buffers(fl_state* st, uint16_t** h, uint16_t** qkv, uint16_t** attn, uint16_t** act);
/* Bound of every inter-workgroup wait inside later decode / verify launches, in ticks of the
 * 100 MHz real-time clock (0: the default, 2 s). A wait that reaches it records FL_E_TIMEOUT and
 * gives up, and so do the launch's later waits; the launch still ends normally, its outputs are
 * then meaningless, and fl_state_check reports the error until fl_state_reset. A tiny bound
 * forces that path from the host (tests of the timeout handling). No counterpart in the
 * reference, whose grid barriers have no bound. */
int fl_state_set_wait_limit(fl_state* st, uint64_t ticks);
/* Tests of the timeout path, no counterpart in the reference: while on != 0, every later decode /
 * verify launch starts (in workgroup 0) with a wait on a word that is never written, so it takes
 * the timeout path once the wait bound is reached, deterministically, and still ends normally. */
int fl_state_force_timeout(fl_state* st, int32_t on);
/* Last error recorded by a kernel (FL_OK or FL_E_TIMEOUT); synchronises the stream. */
int fl_state_check(fl_state* st, void* stream);

/* One full decode step in ONE persistent launch (one workgroup per CU, every workgroup resident
 * at once on an idle device; a plain launch by default, hipLaunchCooperativeKernel when the
 * environment sets FLINT_AMD_COOPERATIVE=1 at fl_state_create; every inter-workgroup wait is
 * bounded either way, see fl_state_set_wait_limit): embedding of *token_in at
 * position pos, all layers, final norm, LM head, greedy argmax (first index on ties over the
 * bf16-rounded logits) written to *token_out. logits (fp32 [V], bf16-exact values) and
 * feat (bf16 [D], post-final-norm hidden) are optional (NULL to skip).
 * token_in / token_out / logits / feat are device pointers.
 * Replaces reference kernels/megakernel_decode.cu:204-237 decode_mega_launch and
 * engine/generate.py:62-66 decode_one_token (greedy). */
int fl_decode_step(const fl_weights* w, fl_state* st, const int32_t* token_in, int32_t pos,
                   int32_t* token_out, float* logits, uint16_t* feat, void* stream);

/* The same decode step with the token SAMPLED in the same launch instead of the greedy argmax:
 * x = bf16(logit / max(temperature, 1e-5)); with 0 < top_k < vocab every x below the top_k-th
 * largest drops out (ties with it stay); p = bf16(softmax(x)); the token is the first index of
 * the largest bf16(p / q), q = bf16(-log u), u from Philox4x32-10 keyed by seed at counter
 * (index, 0, offset low, offset high) — the same steps as fl_sample on this step's logits (the
 * softmax sum runs in another order, so p may differ by a bf16 ulp). vocab <= 65536.
 * Replaces reference engine/generate.py:62-66 decode_one_token with its sample (:52-55:
 * logits_to_probs + multinomial_sample_one_no_sync) fused into the decode step. */
int fl_decode_sample(const fl_weights* w, fl_state* st, const int32_t* token_in, int32_t pos,
                     float temperature, int32_t top_k, uint64_t seed, uint64_t offset,
                     int32_t* token_out, float* logits, uint16_t* feat, void* stream);

/* The same decode step from a hidden state instead of a token: h (device, bf16 [D]) is the
 * layer-0 input as it is (no embedding lookup, no embedding multiplier) and receives the final
 * residual (before the final norm) when the launch completes, in place. token_out (greedy argmax),
 * logits and feat are optional (NULL to skip).
 * Replaces reference kernels/megakernel_decode.cu:204-237 decode_mega_launch(..., h, kc, vc, pos,
 * ...), which takes h (formed on the host as bf16(embed[token] * mult), chat.py:71-74) and mutates
 * it in place (:135, :159). */
int fl_decode_hidden(const fl_weights* w, fl_state* st, uint16_t* h, int32_t pos,
                     int32_t* token_out, float* logits, uint16_t* feat, void* stream);

/* Speculative verify of M tokens in one pass (weights read once for all M):
 * token m sits at cache slot pos+m, RoPE position pos+depth[m]; it attends to the cache
 * [0,pos) plus the slots pos+j with amask[m*M+j] != 0. Writes logits [M,V] (fp32, bf16-exact),
 * argmax per token to tokens_out [M] and feat [M,D] (optional).
 * tokens, depth, amask, tokens_out, logits, feat are device pointers.
 * Replaces reference kernels/verify_mega.cu:246-283 verify_mega_launch. */
int fl_verify(const fl_weights* w, fl_state* st, const int32_t* tokens, int32_t m,
              const int32_t* depth, const uint8_t* amask, int32_t pos,
              int32_t* tokens_out, float* logits, uint16_t* feat, void* stream);

/* KV cache compaction after a tree verify: for i = 0..n-1 (n <= FL_MAX_VERIFY) the K and V rows
 * of cache slot src[i] move to slot dst[i], in every layer and KV group. All n rows are read
 * before any is written, which equals moving them one at a time in order i whenever no source is
 * an earlier move's destination (true of an accepted tree path: src[i] = pos + path[i+1] >=
 * pos + i + 1 = dst[i], path increasing). src / dst are host arrays; n = 0 is a no-op.
 * Replaces the reference's per-step index copies spec_tree.py:124-127. */
int fl_kv_move(fl_state* st, const int32_t* src, const int32_t* dst, int32_t n, void* stream);

/* Temperature / top-k sampling of `rows` logit rows [rows, vocab] (fp32 holding bf16 values, as
 * fl_decode_step / fl_verify write them), vocab <= 65536, one token per row into tokens_out:
 * x = bf16(logit / max(temperature, 1e-5)); with 0 < top_k < vocab every x below the top_k-th
 * largest is dropped (ties with it stay); p = bf16(softmax(x)); the token is the first index of
 * the largest bf16(p / q). q is noise[rows, vocab] when given, else bf16(-log u) with u from
 * Philox4x32-10, key = seed, counter = (index, row, offset low, offset high). probs_out
 * [rows, vocab] (optional) receives p. top_k = 0 means no top-k. Up to 16 rows per launch
 * (more rows: several launches), each row split over up to 64 workgroups that meet at per-row
 * barriers (a plain launch whose grid is checked to fit the device at once: FL_E_LAUNCH if not;
 * cooperative with FLINT_AMD_COOPERATIVE=1); a row whose barrier wait timed out (2 s: a chunk
 * was not resident) gets token -1. The library keeps one scratch block per device (allocated on
 * the first call), so calls on one device must be stream-ordered.
 * Replaces reference engine/generate.py:36-55 (multinomial_sample_one_no_sync, logits_to_probs,
 * sample). */
int fl_sample(const float* logits, int32_t rows, int32_t vocab, float temperature, int32_t top_k,
              uint64_t seed, uint64_t offset, const float* noise, int32_t* tokens_out,
              float* probs_out, void* stream);

/* fl_sample that allocates nothing: the same arguments, results and limits (vocab <= 65536,
 * FL_E_ARG beyond), bit-identical output, but its scratch (per-row histograms, partial sums, the
 * argmax word: 2.1 MB for 16 rows) is a fixed device array of the library, one per GPU,
 * held until the process ends. No hipMalloc, hipFree or allocating library call. Calls on one GPU
 * share that array: calls that overlap on one GPU (other streams or threads) race; keep them
 * stream-ordered. The first call on a device looks the array's address up (no allocation).
 * No counterpart in the reference: for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). */
int fl_sample_noalloc(const float* logits, int32_t rows, int32_t vocab, float temperature,
                      int32_t top_k, uint64_t seed, uint64_t offset, const float* noise,
                      int32_t* tokens_out, float* probs_out, void* stream);

/* ---- diagnostics ------------------------------------------------------------------------ */

/* Hand-off micro-benchmark, no counterpart in the reference (which times its grid barrier in
 * isolation, result.md:38-40): one launch of one 512-thread workgroup per CU hands a tagged
 * vector of `words` 32-bit words (4..8192) from every producer workgroup to every consumer
 * workgroup `rounds` times in a chain, the way the decode / verify kernels hand activations
 * between phases. mode 0: all workgroups, over the uncached exchange memory the kernels use;
 * mode 1: the workgroups of each XCD separately (blockIdx % 8), same memory; mode 2: the
 * workgroups of each XCD over ordinary device memory (coherent loads served by that XCD's L2);
 * modes 0-2 poll single words with a sleep between polls. mode 3 | depth << 8 | gap << 16 |
 * resleep << 24: all workgroups, uncached memory, polled as the decode kernel polls (16-byte
 * groups of 4 words, the missing ones re-requested together) with depth (1..3) rounds of
 * requests in flight, the first rounds gap x 64 cycles apart, resleep x 64 cycles before a
 * re-request; words a multiple of 4. mode 4: the workgroups of each XCD separately, polled as
 * mode 3 with one round in flight.
 * out (device, uint64 [2 * grid]): per workgroup the 100 MHz-clock ticks of all rounds, then its
 * XCC_ID register | (1 << 32) if a wait timed out (0.5 s bound). *grid receives the number of
 * workgroups (the CU count). Stream-ordered; allocates its exchange buffers on the first call. */
int fl_probe_handoff(int32_t mode, int32_t words, int32_t rounds, uint64_t* out, int32_t* grid,
                     void* stream);
/* Compute rate of the exact int4 dequantisation with an M = 8 matrix-core product and no memory
 * traffic, no counterpart in the reference: one 512-thread workgroup per CU, every wave keeping 3
 * units (16 rows x one 128-group) of seeded words in registers and recomputing them `iters`
 * times against 8 token rows in LDS. mode 0: the row layout dequantised on the vector ALUs plus
 * the MFMA dot (k_verify's tile product); mode 1: the tiled layout, dequantisation and dot on
 * the matrix cores (fl_gemv_int4_tiled's unit with token rows). out (device, uint64 [2 * grid]):
 * per workgroup the 100 MHz-clock ticks of its loop, then bits of its result; *grid receives the
 * number of workgroups. Weights per workgroup: 8 x 3 x 2048 x iters. Stream-ordered. */
int fl_probe_dequant(int32_t mode, int32_t iters, uint64_t* out, int32_t* grid, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* FLINT_AMD_H */
