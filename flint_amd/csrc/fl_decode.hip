// Full-model batch-1 decode step as ONE persistent cooperative kernel (gfx950, wave64).
//
// Behaviour follows the reference decode path: kernels/megakernel_decode.cu:164-202 (decode_mega:
// all layers + final norm + LM head in one launch) with the numerics of gpt-fast's forward
// (engine/model.py:134-242): every bf16 rounding point of the reference is reproduced.
//
// Design (MI355X-first, not a translation):
//  * one workgroup of 512 threads per CU; every GEMV phase gives each workgroup a contiguous
//    block of weight rows (one contiguous span of HBM) dealt as 16-byte chunks round-robin over
//    all 512 threads, so every workgroup streams the same number of bytes with fully coalesced
//    loads; per-chunk partials are summed per row in LDS in a fixed order (deterministic);
//  * NO grid barriers: every activation word carries a 16-bit phase tag next to its bf16 value
//    and is exchanged through device-coherent (agent-scope) stores/loads; a consumer polls the
//    words it needs until they carry the producing phase's tag, so one coherence round trip
//    replaces store-completion wait + flag + poll + reload. Every exchange is all-to-all (each
//    phase needs every producer of the previous one), so no workgroup runs more than one phase
//    ahead and buffers need no double-buffering;
//  * the next phase's weight chunks are requested into registers a few at a time between the
//    current phase's chunk computations, after the poll for this phase's inputs (vector loads
//    return in order, so loads issued before a poll would delay it), so the HBM stream overlaps
//    both the compute and the next hand-off;
//  * RMSNorm is recomputed by every workgroup from the residual; RoPE + KV append are fused
//    into the QKV epilogue (NEOX pairs live in adjacent packed rows); SwiGLU into the gate/up
//    epilogue (gate/up rows interleaved); residual adds into the O / down epilogues; greedy
//    argmax into the LM head;
//  * attention: one workgroup per (query head, key slice), the heads of a GQA group on one XCD;
//    its 8 waves take interleaved 8-key steps with an online softmax and merge through LDS;
//    slices (long contexts only) publish tagged partials that slice 0 merges in order.
// The speculative-verify kernel (k_verify, below) runs M tokens through the same protocol with
// the GEMMs on the matrix cores.
#include "fl_common.h"
#include <stdlib.h>
#include <string.h>
#include <mutex>
#include <vector>

namespace {

constexpr int NT = 512;              // threads per workgroup
constexpr int NWAVE = NT / FL_WAVE;  // waves per workgroup
// Chunk budget of one decode-kernel instantiation: the max 16-byte weight chunks per thread in
// each GEMV phase (registers holding one phase's prefetched weights); G3 gate/up chunks
// requested at the start of the O phase's wait and dequantised into registers during it (that
// wait lasts as long as the attention chain); the gate/up chunks requested by then and during
// the O phase (NPRE_GU in all); and PR_GU / PR_D chunks of gate/up and down dequantised into
// registers while the phase's input is exchanged, on top of the PD_* chunks below. A model that
// fits the small budget gets its instantiation: the registers its tighter arrays free hold the
// extra dequantised chunks.
struct ChunksLarge {  // dim <= 3072, inter <= 8192 (any shape the state accepts)
  static constexpr int QKV = 4, O = 4, GU = 12, D = 8, G3 = 0, NPRE_GU = 4, PR_GU = 0, PR_D = 0;
  static constexpr bool ROWS = false;
};
struct ChunksSmall {  // e.g. flint-3b on 256 CUs: 3 / 2 / 10 / 5 chunks per thread
  static constexpr int QKV = 3, O = 2, GU = 10, D = 5, G3 = 4, NPRE_GU = 8, PR_GU = 1, PR_D = 2;
  static constexpr bool ROWS = true;  // QKV and gate/up by rows
};
// chunks per thread dequantised while the phase's input is exchanged: QKV in registers (16 per
// chunk), O, gate/up and down in LDS
constexpr int PD_QKV = 3, PD_O = 2, PD_GU = 3, PD_D = 3;
constexpr int PD_MAX = 3;            // LDS slots: PD_MAX * 64 B per thread
constexpr int MAXC = ChunksLarge::GU;
constexpr int XS_MAX = 8192;         // max staged activation length (bf16 elements)
constexpr int ROWS_MAX = 256;        // max rows per workgroup in one GEMV phase
constexpr int LM_MAXC = 6;           // max 16-byte chunks per lane of one LM-head row (D <= 3072)
constexpr int LM_RB = 2;             // LM-head rows per wave per batch
constexpr int MAX_SLICES = 64;       // attention key slices per kv group
constexpr unsigned long long SPIN_TICKS = 200000000ull;  // default wait bound: 2 s of the 100 MHz realtime clock
// attention LDS (floats): bf16 q / new k / new v rows, then per-wave partials
constexpr int ATT_FLOATS = 96 + NWAVE * 66;
constexpr int WS_FLOATS = (MAXC * NT > ATT_FLOATS) ? MAXC * NT : ATT_FLOATS;

struct DecodeParams {
  fl_weights w;
  uint16_t *kc, *vc;           // [NL, NKV, S, 64] bf16 cache
  uint32_t *h, *attn, *act;    // tagged words: bf16 value | tag << 16
  unsigned long long* qkv;     // tagged NEOX pairs: dim i | dim i+32 << 16 | tag << 32
  unsigned long long* part;    // attention slice partials / verify down-projection parts (tagged fp32)
  unsigned long long* vpart;   // verify attention unit partials (tagged fp32)
  uint16_t *vh, *vattn, *vact; // verify: bf16 [FL_MAX_VERIFY][D | D | F] rows, ready by vflag
  uint32_t* vflag;             // verify: ready flags (tag << 16)
  unsigned long long* amax;    // argmax key
  uint32_t* done;              // final arrivals
  int32_t* err;                // abort flag (spin timeout / bad token)
  const int32_t* token_in;
  int32_t* token_out;
  uint16_t* h_io;              // decode from a hidden state: bf16 [D] input, final residual out
  float* logits;
  uint16_t* feat;
  int D, NH, NKV, F, V, NL, S, pos;
  int att_spw;                 // attention: target 8-key steps per wave per slice
  int gq_min;                  // attention on the matrix cores by KV group from this many cached keys
  int gq_kps;                  // ... with at least this many keys per slice
  int vkps;                    // verify attention: cached keys per slice (a multiple of 16)
  int vtok_work;               // verify attention by tokens while (tokens per unit, 1 for <= 2) x keys <= this
  float eps, emb_mult, attn_scale, resid_mult, logits_scaling;
  uint32_t epoch;              // epoch of this launch's first phase (5 per layer)
  unsigned long long* prof;    // optional per-workgroup phase timestamps (100 MHz clock)
  int prof_slots;
  unsigned long long spin_ticks;  // bound of every inter-workgroup wait (100 MHz ticks)
  const uint32_t* stall;       // tests: when set, workgroup 0 first waits on this never-written word
  // decode only, fused sampling: samp_tdiv > 0 samples the token (temperature divisor
  // max(T, 1e-5), top-k when 0 < samp_topk < V, Philox4x32-10 noise keyed by seed at counter
  // (index, 0, offset)); samp_tdiv = 0 takes the greedy argmax
  float samp_tdiv;
  int samp_topk;
  uint32_t seed_lo, seed_hi, off_lo, off_hi;
  uint32_t* shist;              // [grid][256] tagged per-workgroup histogram counts (count | tag << 16)
  unsigned long long* sword;    // tagged words: [256] bin totals, [grid] maxima, [grid] partial sums
  // verify only: M tokens, their RoPE depths, the [M][M] tree mask, per-token argmax output
  int M;
  const int32_t* tokens;
  const int32_t* depth;
  const uint8_t* amask;
  int32_t* tokens_out;
};

// threadIdx.x / gridDim.x through an empty asm. Index math derived from them is then redone
// where it is used instead of being hoisted out of the layer loop, where dozens of per-chunk
// offsets and predicates would stay live in registers for the whole launch.
__device__ __forceinline__ int tid_here() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int grid_here() {
  int g = gridDim.x;
  asm volatile("" : "+s"(g));
  return g;
}

__device__ __forceinline__ uint32_t tag_of(uint32_t epoch) { return epoch % 65535u + 1u; }

// The launch's parameters read in place from the kernel-argument segment through a pointer the
// compiler cannot follow across the empty asm: each use becomes a scalar load where it is needed
// instead of a value held in an SGPR for the whole layer loop (the kernel's live scalar values
// otherwise exceed the SGPR file and are parked in VGPR lanes, each restore a VALU instruction).
__device__ __forceinline__ const DecodeParams& params_here() {
  typedef const __attribute__((address_space(4))) DecodeParams KParams;
  KParams* k = (KParams*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(k));
  return *(const DecodeParams*)k;
}

__device__ __forceinline__ void row_range(int n, int wg, int G, int& r0, int& rows) {
  int R = (n + G - 1) / G;
  R += (R & 1);
  r0 = wg * R;
  rows = min(R, n - r0);
  if (rows < 0) rows = 0;
}

__device__ __forceinline__ void stamp(const DecodeParams& p, int& slot) {
  if (p.prof && threadIdx.x == 0 && slot < p.prof_slots)
    p.prof[(size_t)blockIdx.x * p.prof_slots + slot] = __builtin_amdgcn_s_memrealtime();
  ++slot;
}

// Slow path of a tag wait: re-read until the tag matches, within a limit of p.spin_ticks (2 s by
// default; no sleep between reads: each sleep of 64 cycles lengthened a hand-off by ~25 ns in the
// hand-off probe, fl_probe.hip mode 3); a timeout (or
// an earlier error) is recorded in p.err and the wait gives up, so a broken producer can never
// hang the GPU. After an error every later wait of the launch gives up within 64 polls.
template <typename T, typename Ok, typename Ld>
__device__ __forceinline__ T spin_until(const DecodeParams& p, T v, Ok ok, Ld ld) {
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  unsigned it = 0;
  while (!ok(v)) {
    v = ld();
    if (__builtin_expect((++it & 63u) == 0, 0)) {  // rare: out of the hot code
      if (__hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > p.spin_ticks) {
        __hip_atomic_store(p.err, (int32_t)FL_E_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  return v;
}

__device__ __forceinline__ unsigned long long wait_pair(const DecodeParams& p,
                                                        const unsigned long long* a, uint32_t tag) {
  auto ld = [a]() { return ld_coh_u64(a); };
  auto ok = [tag](unsigned long long v) { return (uint32_t)(v >> 32) == tag; };
  unsigned long long v = ld();
  if (!ok(v)) v = spin_until(p, v, ok, ld);
  return v;
}

// Poll tagged 64-bit words until every valid one carries `tag`: v[i] holds the last value read of
// word addr(i); the words still missing are re-read together, so each poll costs one round trip
// however many words are missing (a word-by-word wait would pay one per word). Bounded like
// spin_until.
template <int B, typename Addr, typename Valid>
__device__ __forceinline__ void poll_tagged(const DecodeParams& p, unsigned long long (&v)[B],
                                            uint32_t tag, Addr addr, Valid valid) {
  auto ok = [tag](unsigned long long w) { return (uint32_t)(w >> 32) == tag; };
  unsigned long long t0 = 0;
  for (unsigned it = 0;; ++it) {
    bool done = true;
#pragma unroll
    for (int i = 0; i < B; ++i)
      if (valid(i) && !ok(v[i])) done = false;
    if (done) return;
    if (it == 0) t0 = __builtin_amdgcn_s_memrealtime();
#pragma unroll
    for (int i = 0; i < B; ++i)
      if (valid(i) && !ok(v[i])) v[i] = ld_coh_u64(addr(i));
    if (__builtin_expect((it & 63u) == 63u, 0)) {
      if (__hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) return;
      if (__builtin_amdgcn_s_memrealtime() - t0 > p.spin_ticks) {
        __hip_atomic_store(p.err, (int32_t)FL_E_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
    }
  }
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The staged activation vector xs keeps one spare 16-byte slot after every four (logical slot
// s at xslot(s)): a GEMV thread reads the 64 bytes of its chunk's x, and consecutive threads'
// chunks then start 80 bytes apart instead of 64, which spreads a wave's reads over all LDS
// banks instead of a quarter of them.
constexpr int XS_SLOTS = XS_MAX / 8 + XS_MAX / 32;
__device__ __forceinline__ int xslot(int s) { return s + (s >> 2); }

// This thread's 16 bytes of a [D] norm weight vector (D <= 8 * NT: one group per thread),
// requested ahead of the norm so its latency overlaps the wait for the vector being normed.
static_assert(64 * LM_MAXC <= NT, "a norm vector has at most one 16-byte group per thread");
__device__ __forceinline__ uint4 norm_w_load(const uint16_t* __restrict__ nw, int D) {
  return buf_ld128(buf_rsrc(nw, (uint32_t)D * 2u), (uint32_t)tid_here() * 16u);
}

// Second half of RMSNorm (engine/model.py:237-242): xs holds x (bf16), ss the partial sums of
// x^2 of this thread, g this thread's group of the weight (norm_w_load);
// xs <- bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w).
__device__ void norm_finish(float ss, uint4 g, int D, float eps, uint16_t* xs, float* red) {
  const int tid = tid_here();
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  lds_barrier();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) tot += red[w];
  const float r = 1.0f / sqrtf(tot / (float)D + eps);
  const int i = tid;
  if (i < (D >> 3)) {
    const uint4 v = reinterpret_cast<const uint4*>(xs)[xslot(i)];
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float na = rbf(bflo(in[j]) * r), nb = rbf(bfhi(in[j]) * r);
      o[j] = pack_bf16x2(na * bflo(gw[j]), nb * bfhi(gw[j]));
    }
    reinterpret_cast<uint4*>(xs)[xslot(i)] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  lds_barrier();
}

// xs = RMSNorm(bf16(embed_row * mult))  (engine/model.py:138 then :237-242)
__device__ void norm_embed(const uint16_t* __restrict__ erow, float mult,
                           const uint16_t* __restrict__ nw, int D, float eps, uint16_t* xs,
                           float* red) {
  const uint4 g = norm_w_load(nw, D);
  float ss = 0.0f;
  for (int i = tid_here(); i < (D >> 3); i += NT) {
    const uint4 v = reinterpret_cast<const uint4*>(erow)[i];
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = rbf(bflo(in[j]) * mult), b = rbf(bfhi(in[j]) * mult);
      ss += a * a;
      ss += b * b;
      o[j] = pack_bf16x2(a, b);
    }
    reinterpret_cast<uint4*>(xs)[xslot(i)] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  norm_finish(ss, g, D, eps, xs, red);
}

// Stage the tagged vector src[0..n) (n % 4 == 0, n <= XS_MAX) into xs as bf16 once every word
// carries `tag`, and return this thread's sum of squares of its values. Each thread requests
// all of its 16-byte groups at once (coherent range-checked loads, poll_issue) and checks them
// afterwards (poll_wait), so a vector that is already complete costs one round trip, not one
// per group. Work that does not depend on the vector runs between the two while the requests
// are in flight.
constexpr int POLL_MAX = XS_MAX / 4 / NT;     // 16-byte requests per thread for XS_MAX words
constexpr int POLL_D = (64 * 8 * LM_MAXC / 4 + NT - 1) / NT;  // ... for a [D] vector (D <= 64*8*LM_MAXC)
template <int NP>
__device__ __forceinline__ void poll_issue(const uint32_t* src, int n, uint4 (&v)[NP]) {
  const int tid = tid_here();
  const auto rsrc = buf_rsrc(src, (uint32_t)n * 4u);
  asm volatile("" ::: "memory");  // keep the requests after this workgroup's earlier stores
#pragma unroll
  for (int i = 0; i < NP; ++i) v[i] = buf_ld128_coh(rsrc, (uint32_t)(tid + i * NT) * 16u);
}
// A second look at a tagged vector while the wait's work is still running: groups that are
// not yet complete in v are requested again into t (a complete group gets an out-of-range
// request, which touches no memory, so the requests need no branch); poll_merge takes the
// answers in before the wait. By the end of the work the vector has then usually arrived, and
// the wait costs no further round trip.
template <int NP>
struct PollRefresh {
  uint4 t[NP];
  bool need[NP];
  bool issued = false;
};
template <int NP>
__device__ __forceinline__ void poll_refresh(const uint32_t* src, int n, uint32_t tag,
                                             const uint4 (&v)[NP], PollRefresh<NP>& r) {
  const int tid = tid_here();
  const auto rsrc = buf_rsrc(src, (uint32_t)n * 4u);
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int g = tid + i * NT;
    const uint4 w = v[i];
    const bool ok = ((w.x >> 16) == tag) & ((w.y >> 16) == tag) & ((w.z >> 16) == tag) &
                    ((w.w >> 16) == tag);
    r.need[i] = !ok && g < (n >> 2);
    r.t[i] = buf_ld128_coh(rsrc, r.need[i] ? (uint32_t)g * 16u : 0xFFFFFFF0u);
  }
  r.issued = true;
}
template <int NP>
__device__ __forceinline__ void poll_merge(uint4 (&v)[NP], const PollRefresh<NP>& r) {
  if (!r.issued) return;
#pragma unroll
  for (int i = 0; i < NP; ++i)
    if (r.need[i]) v[i] = r.t[i];
}

// Wait until this thread's groups of the tagged vector src[0..n) all carry `tag` (v: the
// requests of poll_issue, refreshed in place); returns the sum of squares of their values
template <int NP>
__device__ __forceinline__ float poll_wait(const DecodeParams& p, const uint32_t* src, int n,
                                           uint32_t tag, uint4 (&v)[NP]) {
  const int tid = tid_here();
  auto ok = [tag](uint4 w) {
    return ((w.x >> 16) == tag) & ((w.y >> 16) == tag) & ((w.z >> 16) == tag) & ((w.w >> 16) == tag);
  };
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int g = tid + i * NT;
    if (g < (n >> 2)) {
      uint4 w = v[i];
      if (!ok(w)) {
        const uint32_t* a = src + 4 * g;
        w = spin_until(p, w, ok, [a]() { return ld_coh_u128(a); });
      }
      v[i] = w;
      const float a0 = bflo(w.x), a1 = bflo(w.y), a2 = bflo(w.z), a3 = bflo(w.w);
      ss += a0 * a0;
      ss += a1 * a1;
      ss += a2 * a2;
      ss += a3 * a3;
    }
  }
  return ss;
}
// xs slots of group g (4 bf16 values: elements 4g .. 4g+3)
__device__ __forceinline__ void xs_put4(uint16_t* xs, int g, uint2 val) {
  reinterpret_cast<uint2*>(xs)[2 * xslot(g >> 1) + (g & 1)] = val;
}
// the values of this thread's groups (v, as poll_wait left them) into xs
template <int NP>
__device__ __forceinline__ void poll_put(int n, uint16_t* xs, const uint4 (&v)[NP]) {
  const int tid = tid_here();
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int g = tid + i * NT;
    const uint4 w = v[i];
    if (g < (n >> 2))
      xs_put4(xs, g, make_uint2((w.x & 0xFFFFu) | (w.y << 16), (w.z & 0xFFFFu) | (w.w << 16)));
  }
}

// The norm weights of this thread's poll groups (group g = tid + i * NT: 4 bf16 weights for
// elements 4g .. 4g+3; groups past D read 0), requested ahead of the norm so their latency
// overlaps the wait for the vector being normed
template <int NP>
__device__ __forceinline__ void norm_w_load4(const uint16_t* __restrict__ nw, int D,
                                             uint2 (&g)[NP]) {
  const auto r = buf_rsrc(nw, (uint32_t)D * 2u);
#pragma unroll
  for (int i = 0; i < NP; ++i) g[i] = buf_ld64(r, (uint32_t)(tid_here() + i * NT) * 8u);
}

// xs = RMSNorm(h) once every word of the tagged residual h carries `tag`; work() runs while the
// first requests for h are in flight
// (engine/model.py:237-242: xs <- bf16(bf16(h * rsqrt(mean(h^2) + eps)) * w)). Each thread
// normalises the groups it polled, from registers: one barrier for the sum of squares, one for xs.
template <typename Work>
__device__ void norm_tagged(const DecodeParams& p, const uint32_t* h, uint32_t tag,
                            const uint16_t* __restrict__ nw, uint16_t* xs, float* red, Work work) {
  const int tid = tid_here();
  uint4 v[POLL_D];
  poll_issue(h, p.D, v);
  uint2 g[POLL_D];
  norm_w_load4(nw, p.D, g);
  PollRefresh<POLL_D> rf;
  work([&] { poll_refresh(h, p.D, tag, v, rf); });
  __builtin_amdgcn_sched_barrier(0);
  poll_merge(v, rf);
  float ss = poll_wait(p, h, p.D, tag, v);
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  lds_barrier();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) tot += red[w];
  const float r = 1.0f / sqrtf(tot / (float)p.D + p.eps);
#pragma unroll
  for (int i = 0; i < POLL_D; ++i) {
    const int gi = tid + i * NT;
    if (gi < (p.D >> 2)) {
      const uint4 w = v[i];
      const float a = rbf(bflo(w.x) * r), b = rbf(bflo(w.y) * r);
      const float c = rbf(bflo(w.z) * r), d = rbf(bflo(w.w) * r);
      xs_put4(xs, gi, make_uint2(pack_bf16x2(a * bflo(g[i].x), b * bfhi(g[i].x)),
                                 pack_bf16x2(c * bflo(g[i].y), d * bfhi(g[i].y))));
    }
  }
  lds_barrier();
}
__device__ void norm_tagged(const DecodeParams& p, const uint32_t* h, uint32_t tag,
                            const uint16_t* __restrict__ nw, uint16_t* xs, float* red) {
  norm_tagged(p, h, tag, nw, xs, red, [](auto&&) {});
}

// xs = values of the tagged vector src[0..n) once all carry `tag` (n <= NP * 4 * NT); work() as
// above
template <int NP, typename Work>
__device__ void stage_tagged(const DecodeParams& p, const uint32_t* src, int n, uint32_t tag,
                             uint16_t* xs, Work work) {
  uint4 v[NP];
  poll_issue(src, n, v);
  PollRefresh<NP> rf;
  work([&] { poll_refresh(src, n, tag, v, rf); });
  __builtin_amdgcn_sched_barrier(0);
  poll_merge(v, rf);
  poll_wait(p, src, n, tag, v);
  lds_barrier();  // every wave is done reading the previous phase's xs
  poll_put(n, xs, v);
  lds_barrier();
}

// Chunk mapping of a GEMV phase. A workgroup's rows [r0, r0+rows) of a [N, K] int4 matrix are
// rows * (K / 32) 16-byte chunks in row-major order (cpr = K / 32 per row), dealt to threads in
// one of two ways:
//  - by stride: thread tid takes chunks f = tid + i * S, i = 0..MC-1, for a stride S <= NT
//    (threads tid >= S take none). S = NT deals them evenly; S = the largest multiple of cpr
//    that is <= NT (cs_stride) keeps each thread in one column of chunks, so it reads its 32
//    activation values once per phase. Partial sums meet in LDS.
//  - by rows: 2^lg lanes per row (rs_lg), lane j of row r takes chunks j + i * 2^lg of row r,
//    so a thread's partial sums add up in a register and a row's sum is a DPP reduction.
//  - by row pairs: 2^lg lanes per pair of rows 2p, 2p+1 (rp_lg); lane j's i-th chunk is chunk
//    j + (i / 2) * 2^lg of row 2p + i % 2, so chunks 2k and 2k+1 of a thread cover the same 32
//    activations: each read of x from LDS serves both rows (gate and up of one output).
// Every mapping gives the four lanes of each 4-lane block the four chunks of one 128-group of one
// row (or all four none), as the matrix-core dequantisation (dq32_mx) needs: cpr is a multiple
// of 4, the strides are multiples of cpr or of NT, and the host admits the by-rows mappings only
// with 2^lg >= 4 lanes per row (phase_fits).
struct ChunkMap {
  bool by_rows;
  int S;    // by stride
  int lg;   // by rows / row pairs
  int cpr, rows;
  bool pairs;
};
__device__ __forceinline__ int cs_stride(int K) {
  const int cpr = K >> 5;
  return (NT / cpr) * cpr;
}
// lanes per row of the by-rows mapping: a power of two <= 32 (the groups of rows 2j and 2j+1
// share a wave), rows * lanes <= NT, and no more lanes than chunks in a row
__device__ __forceinline__ int rs_lg(int rows, int cpr) {
  int lg = 5;
  while (lg > 0 && ((rows << lg) > NT || (1 << (lg - 1)) >= cpr)) --lg;
  return lg;
}
// lanes per row pair: a power of two <= 64, pairs * lanes <= NT, and no more lanes than chunks
__device__ __host__ __forceinline__ int rp_lg(int rows, int cpr) {
  const int pairs = (rows + 1) >> 1;
  int lg = 6;
  while (lg > 0 && ((pairs << lg) > NT || (1 << (lg - 1)) >= cpr)) --lg;
  return lg;
}
__device__ __forceinline__ ChunkMap map_pairs(int K, int rows) {
  return ChunkMap{true, NT, rp_lg(rows, K >> 5), K >> 5, rows, true};
}
__device__ __forceinline__ ChunkMap map_stride(int K, int rows, int S) {
  return ChunkMap{false, S, 0, K >> 5, rows};
}
__device__ __forceinline__ ChunkMap map_rows(int K, int rows) {
  return ChunkMap{true, NT, rs_lg(rows, K >> 5), K >> 5, rows};
}
// chunk index of thread tid's i-th chunk; past every buffer's end where it has none (reads 0)
__device__ __forceinline__ uint32_t chunk_f(const ChunkMap& m, int tid, int i) {
  if (m.by_rows) {
    const int row = m.pairs ? 2 * (tid >> m.lg) + (i & 1) : tid >> m.lg;
    const int c = (tid & ((1 << m.lg) - 1)) + ((m.pairs ? i >> 1 : i) << m.lg);
    return (row < m.rows && c < m.cpr) ? (uint32_t)(row * m.cpr + c) : 0x0FFFFFFFu;
  }
  return tid < m.S ? (uint32_t)(tid + i * m.S) : 0x0FFFFFFFu;
}

// Issue this workgroup's weight chunks for rows [r0, r0+rows) of a [N, K] int4 matrix.
template <int MC>
__device__ __forceinline__ void gemv_load(const uint32_t* __restrict__ q,
                                          const uint32_t* __restrict__ sz, int r0, int rows, int K,
                                          const ChunkMap& m, uint4 (&wr)[MC], uint32_t (&sr)[MC]) {
  const auto wb = buf_rsrc(q + (size_t)r0 * (K >> 3), (uint32_t)rows * (K >> 1));
  const auto sb = buf_rsrc(sz + (size_t)r0 * (K >> 7), (uint32_t)rows * (K >> 5));
  const int tid = tid_here();
#pragma unroll
  for (int i = 0; i < MC; ++i) {  // chunks past this workgroup's rows read as 0
    const uint32_t f = chunk_f(m, tid, i);
    wr[i] = buf_ld128(wb, f * 16u);
    sr[i] = buf_ld32(sb, (f >> 2) * 4u);
  }
}

// The next GEMV phase's weight chunks for rows [r0, r0+rows) of a [N, K] int4 matrix, requested
// a few at a time while this phase computes (a wave that requests a whole phase's chunks at once
// stalls on issue until the memory pipeline drains). on = false requests nothing (empty ranges).
struct NextW {
  __amdgpu_buffer_rsrc_t wb, sb;
  ChunkMap m;  // the next phase's chunk mapping
};
__device__ __forceinline__ NextW next_w(const uint32_t* q, const uint32_t* sz, int r0, int rows,
                                        int K, const ChunkMap& m, bool on) {
  NextW n;
  n.wb = buf_rsrc(q + (size_t)r0 * (K >> 3), on ? (uint32_t)rows * (K >> 1) : 0u);
  n.sb = buf_rsrc(sz + (size_t)r0 * (K >> 7), on ? (uint32_t)rows * (K >> 5) : 0u);
  n.m = m;
  return n;
}
template <int MCN>
__device__ __forceinline__ void next_load(const NextW& n, int j, uint4 (&wn)[MCN],
                                          uint32_t (&sn)[MCN]) {
  const uint32_t f = chunk_f(n.m, tid_here(), j);
  wn[j] = buf_ld128(n.wb, f * 16u);
  sn[j] = buf_ld32(n.sb, (f >> 2) * 4u);
}

// the next phase's chunks [J0, MCN), requested in one go (at the start of that phase)
template <int J0, int MCN>
__device__ __forceinline__ void next_load_from(const NextW& n, uint4 (&wn)[MCN],
                                               uint32_t (&sn)[MCN]) {
#pragma unroll
  for (int j = J0; j < MCN; ++j) next_load(n, j, wn, sn);
}
// ... chunks [J0, J1)
template <int J0, int J1, int MCN>
__device__ __forceinline__ void next_load_range(const NextW& n, uint4 (&wn)[MCN],
                                                uint32_t (&sn)[MCN]) {
#pragma unroll
  for (int j = J0; j < J1; ++j) next_load(n, j, wn, sn);
}

// Dequantise this thread's first PD weight chunks ahead of the x-dots: the dequantisation does
// not depend on the activation vector, so it runs while that vector is still being exchanged
// (the weights arrived during the previous phase). The bf16 results go to this thread's slots
// of dql (uint4 plane k of chunk i at dql[(4i + k) * NT + tid]: conflict-free, and each thread
// reads back only its own slots, so no barrier is needed). Chunks past this workgroup's rows
// read as zero words and scales and dequantise to zeros.
template <int MC, int PD, int OFF = 0, typename Between>
__device__ __forceinline__ void gemv_predq(const uint4 (&wr)[MC], const uint32_t (&sr)[MC],
                                           uint4* dql, Between between) {
  static_assert(PD >= 1 && OFF + PD <= MC && PD <= PD_MAX, "pre-dequantised chunks");
  const int tid = tid_here();
#pragma unroll
  for (int i = 0; i < PD; ++i) {  // chunk OFF + i into slot i
    uint32_t d[4][4];
    dq32_mx(wr[OFF + i], sr[OFF + i], mx_lane(), d);
#pragma unroll
    for (int k = 0; k < 4; ++k) dql[(4 * i + k) * NT + tid] = make_uint4(d[k][0], d[k][1], d[k][2], d[k][3]);
    __builtin_amdgcn_sched_barrier(0);
    between(i);
  }
}

// Register variant for phases with few chunks per thread: d[i] holds chunk OFF + i dequantised.
template <int MC, int PR, int OFF = 0, typename Between>
__device__ __forceinline__ void gemv_predq_reg(const uint4 (&wr)[MC], const uint32_t (&sr)[MC],
                                               uint32_t (&d)[PR][4][4], Between between) {
  static_assert(PR >= 1 && OFF + PR <= MC, "pre-dequantised chunks");
#pragma unroll
  for (int i = 0; i < PR; ++i) {
    dq32_mx(wr[OFF + i], sr[OFF + i], mx_lane(), d[i]);
    __builtin_amdgcn_sched_barrier(0);
    between(i);
  }
}
__device__ __forceinline__ float dq_dot(const uint32_t (&d)[4][4], const uint4* x4) {
  const uint4 x[4] = {x4[0], x4[1], x4[2], x4[3]};
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = dot2_bf16(d[0][i], x[i].x, acc);
    acc = dot2_bf16(d[1][i], x[i].y, acc);
    acc = dot2_bf16(d[2][i], x[i].z, acc);
    acc = dot2_bf16(d[3][i], x[i].w, acc);
  }
  return acc;
}

// dot of a dequantised chunk held in dql with 32 bf16 x values (summed in chunk_dot's order)
__device__ __forceinline__ float dql_dot(const uint4* dql, int i, const uint4* x4) {
  const int tid = tid_here();
  const uint4 x[4] = {x4[0], x4[1], x4[2], x4[3]};
  uint4 d[4];  // plane k: pair k of words 0..3
#pragma unroll
  for (int k = 0; k < 4; ++k) d[k] = dql[(4 * i + k) * NT + tid];
  float acc = 0.0f;
  acc = dot2_bf16(d[0].x, x[0].x, acc);
  acc = dot2_bf16(d[1].x, x[0].y, acc);
  acc = dot2_bf16(d[2].x, x[0].z, acc);
  acc = dot2_bf16(d[3].x, x[0].w, acc);
  acc = dot2_bf16(d[0].y, x[1].x, acc);
  acc = dot2_bf16(d[1].y, x[1].y, acc);
  acc = dot2_bf16(d[2].y, x[1].z, acc);
  acc = dot2_bf16(d[3].y, x[1].w, acc);
  acc = dot2_bf16(d[0].z, x[2].x, acc);
  acc = dot2_bf16(d[1].z, x[2].y, acc);
  acc = dot2_bf16(d[2].z, x[2].z, acc);
  acc = dot2_bf16(d[3].z, x[2].w, acc);
  acc = dot2_bf16(d[0].w, x[3].x, acc);
  acc = dot2_bf16(d[1].w, x[3].y, acc);
  acc = dot2_bf16(d[2].w, x[3].z, acc);
  acc = dot2_bf16(d[3].w, x[3].w, acc);
  return acc;
}

// Lanes per row of the GEMV partial-sum reduction: L = 2^lg with L * rows <= NT and L <= 32, so
// that the groups of rows 2j and 2j+1 share a wave. The lead lane of pair j (the first lane of
// row 2j's group) is lane (2j) << lg. (rows <= ROWS_MAX = NT / 2, so L >= 2.)
__device__ __forceinline__ int row_lanes_lg(int rows) {
  int lg = 5;
  while ((rows << lg) > NT) --lg;
  return lg;
}

// GEMV modes: chunks by stride with partial sums in LDS (GM_STRIDE), the same with each thread
// in one column of chunks (GM_COLUMN: its 32 x values read once, into registers), or by rows
// (GM_ROWS: partial sums in registers, rows summed by DPP; no LDS partials, no barrier).
enum { GM_STRIDE = 0, GM_COLUMN = 1, GM_ROWS = 2, GM_PAIRS = 3 };

// y[r] = sum_k x[k] * dq[r0+r, k] for the chunks loaded by gemv_load with mapping m (mode MODE);
// x staged in xs; chunks i < PD come dequantised ahead: pre_dot(i, x4) is their dot with x.
// After each of this phase's chunks, about 1 / MC of the next phase's chunks [J0, NPRE) are
// requested. Ends with epi(j, y[2j], y[2j+1]) on the lead lane of every row pair j. GM_ROWS
// writes no LDS, and the next writer of xs waits at a barrier of its own; the stride modes end
// with a barrier (part is free again; measured faster than letting the early waves go on).
template <int MC, int MCN, int NPRE, int PD, int MODE, int J0 = 0, typename PreDot, typename Epi>
__device__ __forceinline__ void gemv_compute(const uint4 (&wr)[MC], const uint32_t (&sr)[MC],
                                             PreDot pre_dot, const ChunkMap& m,
                                             const uint16_t* xs, float* part,
                                             const NextW& nx, uint4 (&wn)[MCN],
                                             uint32_t (&sn)[MCN], Epi epi) {
  const int tid = tid_here();
  const int cpr = m.cpr, rows = m.rows;
  auto next = [&](int i) {
#pragma unroll
    for (int j = J0 + i * (NPRE - J0) / MC; j < J0 + (i + 1) * (NPRE - J0) / MC; ++j)
      next_load(nx, j, wn, sn);
  };
  if constexpr (MODE == GM_PAIRS) {  // as GM_ROWS, two rows per lane group over the same chunks
    static_assert(MC % 2 == 0, "chunks come in row pairs");
    const int lg = m.lg, L = 1 << lg;
    const int pr = tid >> lg, lj = tid & (L - 1);
    const bool on = 2 * pr < rows;
    __builtin_amdgcn_s_setprio(1);
    float acc_a = 0.0f, acc_b = 0.0f;
#pragma unroll
    for (int k = 0; k < MC / 2; ++k) {
      const int c = lj + (k << lg);
      const uint4* x4 = reinterpret_cast<const uint4*>(xs) + xslot(4 * min(c, cpr - 1));
      const uint4 xr[4] = {x4[0], x4[1], x4[2], x4[3]};  // read once for both rows
      const int i = 2 * k;
      const bool ok = on && c < cpr;
      const float ya = (i < PD) ? pre_dot(i, xr) : chunk_dot_mx(wr[i], sr[i], xr, 0.0f);
      acc_a += ok ? ya : 0.0f;
      next(i);
      __builtin_amdgcn_sched_barrier(0);  // one chunk's temporaries live at a time
      const float yb = (i + 1 < PD) ? pre_dot(i + 1, xr) : chunk_dot_mx(wr[i + 1], sr[i + 1], xr, 0.0f);
      acc_b += ok ? yb : 0.0f;
      next(i + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    acc_a = group_sum(acc_a, L);
    acc_b = group_sum(acc_b, L);
    if (on && lj == 0) epi(pr, acc_a, acc_b);
    __builtin_amdgcn_s_setprio(0);
    return;
  }
  if constexpr (MODE == GM_ROWS) {
    const int lg = m.lg, L = 1 << lg;
    const int row = tid >> lg, lj = tid & (L - 1);
    const bool on = row < rows;
    // Waves still in this phase issue first: a wave that has finished its rows goes on to the
    // next phase's dequantisation, which would otherwise take the shared SIMD from the waves
    // whose rows everyone waits for (s_setprio: the wave's own issue priority).
    __builtin_amdgcn_s_setprio(1);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < MC; ++i) {
      const int c = lj + (i << lg);
      const uint4* x4 = reinterpret_cast<const uint4*>(xs) + xslot(4 * min(c, cpr - 1));
      const float y = (i < PD) ? pre_dot(i, x4) : chunk_dot_mx(wr[i], sr[i], x4, 0.0f);
      acc += (on && c < cpr) ? y : 0.0f;
      next(i);
      __builtin_amdgcn_sched_barrier(0);  // one chunk's temporaries live at a time; loads spread
    }
    acc = group_sum(acc, L);  // every lane of the row's group holds the row's sum
    const float other = __shfl_xor(acc, L);
    if (on && !(row & 1) && lj == 0) epi(row >> 1, acc, other);
    __builtin_amdgcn_s_setprio(0);
    return;
  }
  const int S = m.S;
  const int total = rows * cpr;
  const bool active = tid < S;
  __builtin_amdgcn_s_setprio(1);  // as in GM_ROWS, until this phase's sums are out
  if constexpr (MODE == GM_COLUMN) {
    const uint4* xp = reinterpret_cast<const uint4*>(xs) + xslot(4 * (tid % cpr));
    const uint4 xr[4] = {xp[0], xp[1], xp[2], xp[3]};
#pragma unroll
    for (int i = 0; i < MC; ++i) {
      const int f = tid + i * S;
      if (active && f < total)
        part[f] = (i < PD) ? pre_dot(i, xr) : chunk_dot_mx(wr[i], sr[i], xr, 0.0f);
      next(i);
      __builtin_amdgcn_sched_barrier(0);  // one chunk's temporaries live at a time
    }
  } else {
    int c = tid % cpr;
    const int step = S % cpr;
#pragma unroll
    for (int i = 0; i < MC; ++i) {
      const int f = tid + i * S;
      const uint4* x4 = reinterpret_cast<const uint4*>(xs) + xslot(4 * c);
      if (active && f < total)
        part[f] = (i < PD) ? pre_dot(i, x4) : chunk_dot_mx(wr[i], sr[i], x4, 0.0f);
      c += step;
      if (c >= cpr) c -= cpr;
      next(i);
      __builtin_amdgcn_sched_barrier(0);  // one chunk's temporaries live at a time; loads spread
    }
  }
  lds_barrier();
  // per row, L = 2^lg lanes each sum every L-th partial, four requests at a time (one LDS round
  // trip per four partials), in the same order as a sequential loop
  const int lg = row_lanes_lg(rows);
  const int L = 1 << lg;
  const int row = tid >> lg, li = tid & (L - 1);
  float acc = 0.0f;
  if (row < rows) {
    const float* pr = part + row * cpr;
    for (int j0 = li; j0 < cpr; j0 += 4 * L) {
      float v[4];
#pragma unroll
      for (int m4 = 0; m4 < 4; ++m4) v[m4] = pr[min(j0 + m4 * L, cpr - 1)];
#pragma unroll
      for (int m4 = 0; m4 < 4; ++m4) acc += (j0 + m4 * L < cpr) ? v[m4] : 0.0f;
    }
  }
  acc = group_sum(acc, L);  // every lane of the row's group holds the row's sum
  // rows 2j and 2j+1 are neighbouring groups of one wave (L <= 32): the first lane of row 2j
  // runs the pair's epilogue from registers, before the barrier that frees `part`. (ds_bpermute
  // measured faster here than the DPP / permlane exchanges of the same lanes.)
  const float other = __shfl_xor(acc, L);
  if (row < rows && !(row & 1) && li == 0) epi(row >> 1, acc, other);
  lds_barrier();
  __builtin_amdgcn_s_setprio(0);
}

// Key slices of one query head over the cached keys 0..pos-1. Keys are processed in 8-key steps
// (8 keys x 64 dims: one 16-byte K load and one 16-byte V load per lane); a slice is one
// workgroup, whose 8 waves take interleaved steps so that each group of 8 steps covers 64
// consecutive keys. One slice while no wave takes more than `spw` steps; beyond that, 4/5 of the
// workgroups take a slice each (NH x nsl <= 0.8 G), at most G / NH and MAX_SLICES, at least 1 (the
// new key at pos always has a slice). Measured at flint-3b (40 heads, 256 workgroups; tok/s by
// slice count, the merge left to the O phase from 2 slices): ctx 128 / 256: 1 slice 1165 / 1141
// against 1128-1133 / 1124-1130 with 3-5; ctx 512 / 1024 / 2048 / 4096: 5 slices 1121 / 1109 /
// 1069 / 981 against 2 slices 1095 / 1035 (merged in the attention phase), 6 slices 1093 / 1081 /
// 1055 / 971, 4 slices 1116 / 1100 / 1027 / 943. spw < 0 fixes the count at -spw (tuning knob).
__host__ __device__ inline void attn_slices(int pos, int NH, int G, int spw, int& nsl, int& sps) {
  const int ns = (pos + 7) >> 3;
  if (spw < 0)
    nsl = -spw;
  else if (ns <= NWAVE * spw)
    nsl = 1;
  else
    nsl = (4 * G) / (5 * NH);
  if (nsl < 1) nsl = 1;
  int cap = G / NH < MAX_SLICES ? G / NH : MAX_SLICES;
  if (cap < 1) cap = 1;
  if (nsl > cap) nsl = cap;
  sps = (ns + nsl - 1) / nsl;
  nsl = sps > 0 ? (ns + sps - 1) / sps : 1;
  if (nsl < 1) nsl = 1;
}

// GQA flash-decode attention of one layer (engine/model.py:171-179: q.k^T * scale, softmax and
// p.v in fp32 over keys 0..pos, bf16 output; head h reads kv group h / (NH / NKV)).
// One workgroup per (query head, key slice): u = (j * nsl + sl) * NKV + g for head j of kv group
// g, so all heads of a group run on workgroups u = g (mod NKV) -- with NKV = 8 and workgroups
// dealt round-robin over the 8 XCDs, a group's K/V rows are fetched into one L2. At short
// contexts every head is one slice, so no workgroup waits for another.
// Lane (kk = lane / 8, ds = lane % 8) of a wave holds dims 8ds..8ds+7 of key kk of each step:
// q . k is 4 dot2 plus a 3-step DPP sum over the key's 8 lanes, p.v is 8 FMAs, and the output
// is summed over the 8 keys once at the end. The slice's cached K / V rows (keys < pos) are
// requested before the wait for this launch's q, so the cache reads overlap it. The new key
// (position pos, appended to the cache by this same launch) comes from the tagged q/k/v words
// and is folded in by wave 0 of slice 0 as one extra key. Softmax uses the exact max of each
// round of steps with an online rescale between rounds and for the new key. Waves merge through
// LDS; slices > 0 publish (m, l, o) as tagged 64-bit words and slice 0 merges them in order (with
// DEFER_MERGE_SLICES or more slices it returns its own (m, l, o) in mg and merges in the O phase).
// With this many key slices or more (the host's default; FLINT_AMD_DEFER_SLICES to tune), slice 0
// leaves its merge to the O phase, after its own O chunks are dequantised (it waits longest for the
// other slices, and its workgroup would otherwise start that work last and be the last O
// producer). Measured against merging in the attention phase: ctx 2048 / 3072 / 4096 / 8192 (4, 6,
// 6, 6 slices): -24, -66, -40, -48 us per step; at ctx 512 with 2 slices +10 tok/s (1105 against
// 1095) once the GEMVs dequantised on the matrix cores (before that, +30 us per step).
constexpr int DEFER_MERGE_SLICES = 2;
// A key-slice merge left to the caller: slice 0's (max, sum, o) after its own keys (wave 0, lane d)
struct SliceMerge {
  bool pend = false;  // workgroup-uniform
  float M, Ls, O;
  int hq, nsl;
};
// slice 0 of head hq folds in slices 1 .. nsl-1 in order (online rescale), four slices per batch,
// and writes the head's output; run by wave 0 (lane d: output dim d)
__device__ __forceinline__ void slice_merge(const DecodeParams& p, const SliceMerge& mg, uint32_t otag,
                                            uint32_t ptag) {
  const int d = tid_here();
  float M = mg.M, Ls = mg.Ls, O = mg.O;
  const int nsl = mg.nsl;
  const unsigned long long* hpart = p.part + (size_t)mg.hq * MAX_SLICES * 66;
  for (int c0 = 1; c0 < nsl; c0 += 4) {
    unsigned long long wm[4], wl[4], wo[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const unsigned long long* cp = hpart + (size_t)min(c0 + b, nsl - 1) * 66;
      wm[b] = ld_coh_u64(cp);
      wl[b] = ld_coh_u64(cp + 1);
      wo[b] = ld_coh_u64(cp + 2 + d);
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (c0 + b >= nsl) break;
      const unsigned long long* cp = hpart + (size_t)(c0 + b) * 66;
      auto ok = [ptag](unsigned long long v) { return (uint32_t)(v >> 32) == ptag; };
      if (!ok(wm[b])) wm[b] = spin_until(p, wm[b], ok, [cp]() { return ld_coh_u64(cp); });
      if (!ok(wl[b])) wl[b] = spin_until(p, wl[b], ok, [cp]() { return ld_coh_u64(cp + 1); });
      if (!ok(wo[b]))
        wo[b] = spin_until(p, wo[b], ok, [cp, d]() { return ld_coh_u64(cp + 2 + d); });
      const float mc = __uint_as_float((uint32_t)wm[b]);
      const float Mn = fmaxf(M, mc);
      const float ea = __builtin_amdgcn_exp2f(M - Mn), eb = __builtin_amdgcn_exp2f(mc - Mn);
      Ls = Ls * ea + __uint_as_float((uint32_t)wl[b]) * eb;
      O = O * ea + __uint_as_float((uint32_t)wo[b]) * eb;
      M = Mn;
    }
  }
  st_coh_u32(p.attn + mg.hq * 64 + d, f2bf(O / Ls) | (otag << 16));
}

// DEFER: the kernel instantiation that leaves slice 0's merge to the O phase from
// DEFER_MERGE_SLICES slices on (the other one merges here whatever the slice count)
template <bool DEFER>
__device__ void attention_phase(const DecodeParams& p, int l, uint32_t qtag, uint32_t otag,
                                uint32_t ptag, float* ws, int& slot, SliceMerge& mg) {
  // steps per wave per round, in groups of RG: a group whose first step lies past the slice is
  // skipped. Groups of 2 measured best (against 4: -4 to -10 us per step at ctx 512-1024, -16 at
  // 2048, -12 at 8192; groups of 1 lose at long contexts)
  constexpr int RG = 2, NG = 4, RB = RG * NG;
  const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
  const int kk = lane >> 3, ds = lane & 7;
  const int pos = p.pos;
  const int ns = (pos + 7) >> 3;
  int nsl, sps;
  attn_slices(pos, p.NH, grid_here(), p.att_spw, nsl, sps);
  const int u = blockIdx.x;
  if (u >= p.NH * nsl) {
    stamp(p, slot);
    stamp(p, slot);
    stamp(p, slot);
    return;
  }
  const int g = u % p.NKV, rest = u / p.NKV, sl = rest % nsl, j = rest / nsl;
  const int hq = g * (p.NH / p.NKV) + j;
  const int s0 = sl * sps, s1 = min(ns, s0 + sps);
  const int nrounds = (s1 - s0 + NWAVE * RB - 1) / (NWAVE * RB);
  // this slice's cached rows: keys [8 s0, min(8 s1, pos)); loads outside read as 0
  const int k0 = s0 * 8, k1 = min(s1 * 8, pos);
  const size_t cbase = ((size_t)(l * p.NKV + g) * p.S + k0) * 64;
  const uint32_t kbytes = (uint32_t)max(k1 - k0, 0) * 128u;
  const auto kb = buf_rsrc(p.kc + cbase, kbytes);
  const auto vb = buf_rsrc(p.vc + cbase, kbytes);

  uint4 kr[RB], vr[RB];
  auto step_of = [&](int r, int i) { return s0 + r * NWAVE * RB + wave + NWAVE * i; };
  auto issue = [&](int r) {
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const uint32_t off = (uint32_t)((step_of(r, i) * 8 + kk - k0) * 128 + ds * 16);
      kr[i] = buf_ld128(kb, off);
      vr[i] = buf_ld128(vb, off);
    }
  };
  if (nrounds > 0) issue(0);

  // LDS: bf16 [3][64]: q of head hq, this step's new k and v of group g
  uint16_t* qs = reinterpret_cast<uint16_t*>(ws);
  float* wpart = ws + 96;  // [NWAVE][66]: m, l, o[64] per wave
  if (tid < 96) {
    const int r = tid >> 5, jj = tid & 31;
    const int hh = r == 0 ? hq : (r == 1 ? p.NH + g : p.NH + p.NKV + g);
    const unsigned long long v = wait_pair(p, p.qkv + hh * 32 + jj, qtag);
    qs[r * 64 + jj] = (uint16_t)v;               // NEOX pair: dim jj ...
    qs[r * 64 + jj + 32] = (uint16_t)(v >> 16);  // ... and dim jj + 32
  }
  lds_barrier();
  stamp(p, slot);
  const uint32_t* qs32 = reinterpret_cast<const uint32_t*>(ws);
  uint32_t qv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) qv[e] = qs32[ds * 4 + e];
  // scores in the log2 domain: p = 2^(s * scale * log2(e) - m)
  const float sc = p.attn_scale * 1.4426950408889634f;

  float m = -INFINITY, lsum = 0.0f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;
  for (int r = 0; r < nrounds; ++r) {
    if (r > 0) issue(r);
    float s[RB];
    float rmax = -INFINITY;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      if (step_of(r, gi * RG) < s1) {
#pragma unroll
        for (int ii = 0; ii < RG; ++ii) {
          const int i = gi * RG + ii;
          const int st = step_of(r, i);
          float a = dot2_bf16(kr[i].x, qv[0], 0.0f);
          a = dot2_bf16(kr[i].y, qv[1], a);
          a = dot2_bf16(kr[i].z, qv[2], a);
          a = dot2_bf16(kr[i].w, qv[3], a);
          a = sum8(a);
          s[i] = (st < s1 && st * 8 + kk < pos) ? a * sc : -INFINITY;
          rmax = fmaxf(rmax, s[i]);
        }
      }
    }
    const float mn = fmaxf(m, max_stride8(rmax));
    const float mu = (mn == -INFINITY) ? 0.0f : mn;  // no valid key yet: every p is 0
    const float corr = __builtin_amdgcn_exp2f(m - mu);  // 0 while m = -inf
    lsum *= corr;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= corr;
    m = mn;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      if (step_of(r, gi * RG) < s1) {
#pragma unroll
        for (int ii = 0; ii < RG; ++ii) {
          const int i = gi * RG + ii;
          const float pw = __builtin_amdgcn_exp2f(s[i] - mu);
          lsum += pw;
          o[0] = __builtin_fmaf(pw, bflo(vr[i].x), o[0]);
          o[1] = __builtin_fmaf(pw, bfhi(vr[i].x), o[1]);
          o[2] = __builtin_fmaf(pw, bflo(vr[i].y), o[2]);
          o[3] = __builtin_fmaf(pw, bfhi(vr[i].y), o[3]);
          o[4] = __builtin_fmaf(pw, bflo(vr[i].z), o[4]);
          o[5] = __builtin_fmaf(pw, bfhi(vr[i].z), o[5]);
          o[6] = __builtin_fmaf(pw, bflo(vr[i].w), o[6]);
          o[7] = __builtin_fmaf(pw, bfhi(vr[i].w), o[7]);
        }
      }
    }
  }
  if (sl == 0 && wave == 0) {  // the new key / value at pos (lanes kk = 0 carry its p)
    float a = dot2_bf16(qs32[32 + ds * 4], qv[0], 0.0f);
    a = dot2_bf16(qs32[32 + ds * 4 + 1], qv[1], a);
    a = dot2_bf16(qs32[32 + ds * 4 + 2], qv[2], a);
    a = dot2_bf16(qs32[32 + ds * 4 + 3], qv[3], a);
    const float sn = sum8(a) * sc;
    const float mn = fmaxf(m, sn);
    const float corr = __builtin_amdgcn_exp2f(m - mn);  // 0 while m = -inf
    const float pn = (kk == 0) ? __builtin_amdgcn_exp2f(sn - mn) : 0.0f;
    lsum = lsum * corr + pn;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t vw = qs32[64 + ds * 4 + e];
      o[2 * e] = __builtin_fmaf(pn, bflo(vw), o[2 * e] * corr);
      o[2 * e + 1] = __builtin_fmaf(pn, bfhi(vw), o[2 * e + 1] * corr);
    }
    m = mn;
  }
  stamp(p, slot);
  // sum over the 8 keys of a step (lanes kk = 0..7 with the same ds), then merge the waves
  lsum = sum_stride8(lsum);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = sum_stride8(o[e]);
  float* mywp = wpart + wave * 66;
  if (kk == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) mywp[2 + ds * 8 + e] = o[e];
  }
  if (lane == 0) {
    mywp[0] = m;
    mywp[1] = lsum;
  }
  lds_barrier();
  // The merge runs in wave 0 at raised issue priority; the other waves go on to the next phase's
  // dequantisation meanwhile (no barrier at the end: that phase touches only each thread's own
  // dql slots before a barrier of its own, and the LDS used here only after it).
  if (tid < 64) __builtin_amdgcn_s_setprio(1);
  if (tid < 64) {  // thread d: output dim d, waves merged in a fixed order
    const int d = tid;
    // every wave's values are read before any is used: one LDS round trip instead of one per
    // wave's output value (+0.7% tok/s at ctx 512, measured on one box)
    float M = -INFINITY, Ls = 0.0f, O = 0.0f;
    float wmx[NWAVE], wls[NWAVE], wov[NWAVE];
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      wmx[w] = wpart[w * 66];
      wls[w] = wpart[w * 66 + 1];
      wov[w] = wpart[w * 66 + 2 + d];
    }
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, wmx[w]);
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const float e = (wmx[w] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(wmx[w] - M);
      Ls += wls[w] * e;
      O += wov[w] * e;
    }
    unsigned long long* hpart = p.part + (size_t)hq * MAX_SLICES * 66;
    if (sl > 0) {
      // publish this slice's (m, l, o) as tagged words: fp32 bits | 32-bit tag << 32
      unsigned long long* pp = hpart + (size_t)sl * 66;
      const unsigned long long tg = (unsigned long long)ptag << 32;
      if (d == 0) {
        st_coh_u64(pp, (unsigned long long)__float_as_uint(M) | tg);
        st_coh_u64(pp + 1, (unsigned long long)__float_as_uint(Ls) | tg);
      }
      st_coh_u64(pp + 2 + d, (unsigned long long)__float_as_uint(O) | tg);
    } else {
      mg.M = M;
      mg.Ls = Ls;
      mg.O = O;
      mg.hq = hq;
      mg.nsl = nsl;
      if (!DEFER || nsl < 2) slice_merge(p, mg, otag, ptag);
    }
  }
  mg.pend = DEFER && sl == 0 && nsl >= 2;
  __builtin_amdgcn_s_setprio(0);
  stamp(p, slot);
}

// ---- long-context decode attention on the matrix cores, by KV group ----------------------------
// One unit per (KV group g, key slice): the group's QPG query heads are the rows of the MFMA
// tiles (engine/model.py:210-212 repeats the group's K / V for them; here the K / V rows are read
// once for all QPG heads). Per 16-key chunk S^T = K Q^T with two 16x16x32 bf16 MFMAs, an online
// softmax per head (exp2 domain), O^T = V^T P^T with 16x16x16 bf16 MFMAs and P split into three
// bf16 terms (each product with a bf16 value exact in fp32): the same arithmetic as the verify
// kernel's slice units, for one token. K rows and V^T go through LDS in rounds of GQ_VRK keys
// (the first requested before the q wait); the last slice also takes the new key at pos. The 8
// waves take interleaved chunks and merge through LDS. With one slice per group a unit writes
// its heads' outputs; otherwise every unit publishes each head's (max, sum, o) as tagged fp32
// words and the unit of slice s merges the heads j = s (mod nsl) over the slices (gqa_merge: in
// a fixed order, so the result is deterministic). Units are numbered u = s * NKV + g, so a
// group's slices run on workgroups of one XCD. The k_decode<C, 2> instantiation, which the host
// picks from p.gq_min cached keys on (gqa_applies; off by default: the per-head kernels measure as
// fast or faster up to 16 K keys on flint-3b), with slices of at least p.gq_kps = 128 keys (at
// most 32 per group). Rounds of 288 keys keep one round per slice up to ctx 9216: with 256 a
// context just past 8192 took a second, nearly empty round (+52 us at 8320; 288 costs ~4 us below).
constexpr int GQ_VRK = 288;                      // keys per LDS round (32 slices x 288 keys: one round up to ctx 9216)
constexpr int GQ_VT_LD = GQ_VRK + 8;             // V^T row pitch (bf16)
constexpr int GQ_CPT = (GQ_VRK * 8 + NT - 1) / NT;  // 16-byte K (and V) chunks per thread per round
constexpr int GQ_KT = NT - FL_WAVE;                   // threads of the first round (all waves but the last)
constexpr int GQ_CPT1 = (GQ_VRK * 8 + GQ_KT - 1) / GQ_KT;  // ... and their chunks each
static_assert(GQ_CPT1 >= GQ_CPT, "the register arrays hold either kind of round");
constexpr int GQ_ROWS = 8;                       // query heads per KV group this path takes
constexpr int GQ_MAXSL = 32;                     // slices per group (4 per wave in the merge)
constexpr int GQ_KS = 0, GQ_VT = GQ_KS + GQ_VRK * 128, GQ_WP = GQ_VT + 64 * GQ_VT_LD * 2;
constexpr int GQ_BYTES = GQ_WP + NWAVE * GQ_ROWS * 66 * 4;
static_assert(GQ_BYTES <= PD_MAX * 4 * NT * 16, "the GQA attention's LDS lives in the dequantised-chunk slots");
static_assert((16 + 2) * 64 * 2 <= WS_FLOATS * 4, "q rows and the new key in ws");

__device__ __forceinline__ void gqa_slices(int pos, int NKV, int G, int kps, int& nsl, int& spk) {
  nsl = max(1, min(min(GQ_MAXSL, G / NKV), (pos + kps - 1) / kps));
  spk = (pos + nsl - 1) / nsl;
  nsl = max(1, (pos + spk - 1) / spk);
}
// whether a decode launch takes the attention by KV group (the host picks the k_decode
// instantiation that holds it by the same rule)
__host__ __device__ inline bool gqa_applies(int pos, int gq_min, int NH, int NKV, int G) {
  return pos >= gq_min && NH / NKV <= GQ_ROWS && NKV <= G;
}

// The unit of slice sl of KV group g merges the group's heads j = sl, sl + nsl, ... over the nsl
// slices' published (max, sum, o): wave w takes slices w, w + 8, w + 16, w + 24 (lane d: their max,
// sum and o[d], one batch), the waves' results meet in wp (NWAVE x 66 floats of LDS) and wave 0
// combines them in wave order. Every thread of the workgroup calls it (it has barriers).
__device__ void gqa_merge(const DecodeParams& p, int g, int sl, int nsl, float* wp, uint32_t otag,
                        uint32_t ptag) {
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  const int QPG = p.NH / p.NKV;
  for (int j = sl; j < QPG; j += nsl) {
    const int d = lane;
    const unsigned long long* hp = p.part + (size_t)(g * QPG + j) * MAX_SLICES * 66;
    constexpr int SPW = GQ_MAXSL / NWAVE;
    unsigned long long wv[3 * SPW];
    auto valid = [&](int i) { return wave + NWAVE * (i / 3) < nsl; };
    auto addr = [&](int i) {
      const int sidx = min(wave + NWAVE * (i / 3), nsl - 1), k = i % 3;
      return hp + (size_t)sidx * 66 + (k == 2 ? 2 + d : k);
    };
#pragma unroll
    for (int i = 0; i < 3 * SPW; ++i) wv[i] = valid(i) ? ld_coh_u64(addr(i)) : 0ull;
    poll_tagged<3 * SPW>(p, wv, ptag, addr, valid);
    float M = -INFINITY, L = 0.0f, O = 0.0f;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {  // this wave's slices in order (online rescale)
      if (wave + NWAVE * k < nsl) {
        const float mc = __uint_as_float((uint32_t)wv[3 * k]);
        const float Mn = fmaxf(M, mc);
        const float ea = (M == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
        const float eb = (mc == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mc - Mn);
        L = L * ea + __uint_as_float((uint32_t)wv[3 * k + 1]) * eb;
        O = O * ea + __uint_as_float((uint32_t)wv[3 * k + 2]) * eb;
        M = Mn;
      }
    }
    float* w = wp + wave * 66;
    if (d == 0) {
      w[0] = M;
      w[1] = L;
    }
    w[2 + d] = O;
    lds_barrier();
    if (wave == 0) {
      float MM = -INFINITY, LL = 0.0f, OO = 0.0f;
      for (int q = 0; q < NWAVE; ++q) MM = fmaxf(MM, wp[q * 66]);
      for (int q = 0; q < NWAVE; ++q) {
        const float* x = wp + q * 66;
        const float e = (x[0] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(x[0] - MM);
        LL += x[1] * e;
        OO += x[2 + d] * e;
      }
      st_coh_u32(p.attn + (g * QPG + j) * 64 + d, f2bf(OO / LL) | (otag << 16));
    }
    lds_barrier();  // wp is free again
  }
}

__device__ void attention_gqa(const DecodeParams& p, int l, uint32_t qtag, uint32_t otag,
                              uint32_t ptag, float* ws, unsigned char* ua, int& slot) {
  const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, c = lane >> 4;
  const int pos = p.pos, NH = p.NH, NKV = p.NKV, QPG = NH / NKV;
  int nsl, spk;
  gqa_slices(pos, NKV, grid_here(), p.gq_kps, nsl, spk);
  const int u = blockIdx.x;
  if (u >= NKV * nsl) {
    stamp(p, slot);
    stamp(p, slot);
    stamp(p, slot);
    return;
  }
  const int g = u % NKV, sl = u / NKV;
  const bool last = sl == nsl - 1;  // also takes the new key
  const int k0 = sl * spk, nc = max(0, min(pos, k0 + spk) - k0);
  const size_t cbase = (size_t)(l * NKV + g) * p.S * 64;
  uint16_t* const ks = reinterpret_cast<uint16_t*>(ua + GQ_KS);
  uint16_t* const vt = reinterpret_cast<uint16_t*>(ua + GQ_VT);
  float* const wp = reinterpret_cast<float*>(ua + GQ_WP);
  uint16_t* const qs = reinterpret_cast<uint16_t*>(ws);  // [16][64] q rows, then new k, new v
  uint16_t* const kn = qs + 16 * 64;
  uint16_t* const vn = kn + 64;
  // cached keys [k0 + kb, k0 + kb + n): requested into registers by NTH threads, CPT 16-byte
  // chunks each (request_round), then stored into rows 0 .. n-1 of ks and columns 0 .. n-1 of vt
  // (store_round)
  uint4 kv[GQ_CPT1], vv[GQ_CPT1];
  auto request_round = [&](int kb, int n, auto cpt, int nth) {
    const auto kr = buf_rsrc(p.kc + cbase + (size_t)(k0 + kb) * 64, (uint32_t)n * 128u);
    const auto vr = buf_rsrc(p.vc + cbase + (size_t)(k0 + kb) * 64, (uint32_t)n * 128u);
#pragma unroll
    for (int i = 0; i < decltype(cpt)::value; ++i) {  // loads past the round's n keys read as 0, touching no memory
      const int ci = tid + nth * i;
      kv[i] = buf_ld128(kr, (uint32_t)ci * 16u);
      vv[i] = buf_ld128(vr, (uint32_t)ci * 16u);
    }
  };
  auto store_round = [&](int n, auto cpt, int nth) {
#pragma unroll
    for (int i = 0; i < decltype(cpt)::value; ++i) {
      const int ci = tid + nth * i, key = ci >> 3, d0 = (ci & 7) * 8;
      if (key >= n) continue;  // a row past the round: the new key may be staged there
      *reinterpret_cast<uint4*>(ks + key * 64 + d0) = kv[i];
      const uint32_t w4[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt[(d0 + 2 * e) * GQ_VT_LD + key] = (uint16_t)w4[e];
        vt[(d0 + 2 * e + 1) * GQ_VT_LD + key] = (uint16_t)(w4[e] >> 16);
      }
    }
  };
  using CptAll = std::integral_constant<int, GQ_CPT>;
  using CptKey = std::integral_constant<int, GQ_CPT1>;
  auto load_round = [&](int kb, int n) {  // later rounds: every thread
    request_round(kb, n, CptAll{}, NT);
    store_round(n, CptAll{}, NT);
  };
  // The first round of cached keys is requested by the seven key waves before the q wait and
  // stored after it; the last wave holds no keys and polls q (and the new k / v) alone. A wave's
  // loads complete in order, so a poll behind a wave's share of the round (72 KB per workgroup)
  // returned only after the round had arrived: the q / k / v wait took 4.0-4.4 us per layer at
  // ctx 8192 against 2.1 us in the per-head units.
  const bool keyw = wave < NWAVE - 1;
  if (nc > 0 && keyw) request_round(0, min(nc, GQ_VRK), CptKey{}, GQ_KT);
  if (!keyw) {  // q of the group's heads (rows 0 .. QPG-1) and, for the last slice, the new key's k and v
    const int nq = QPG * 32, total = nq + (last ? 64 : 0);
    constexpr int B = (GQ_ROWS * 32 + 64 + 63) / 64;
    auto word = [&](int idx) {
      if (idx < nq) return p.qkv + (g * QPG + (idx >> 5)) * 32 + (idx & 31);
      const int i2 = idx - nq;
      return p.qkv + ((i2 >> 5) ? NH + NKV + g : NH + g) * 32 + (i2 & 31);
    };
    unsigned long long v[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int idx = lane + i * 64;
      v[i] = idx < total ? ld_coh_u64(word(idx)) : 0ull;
    }
    poll_tagged<B>(p, v, qtag, [&](int i) { return word(lane + i * 64); },
                   [&](int i) { return lane + i * 64 < total; });
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int idx = lane + i * 64;
      if (idx < total) {
        uint16_t* dst = idx < nq ? qs + (idx >> 5) * 64 : ((idx - nq) >> 5 ? vn : kn);
        const int dp = idx & 31;  // NEOX pair: dims dp and dp + 32
        dst[dp] = (uint16_t)v[i];
        dst[dp + 32] = (uint16_t)(v[i] >> 16);
      }
    }
    for (int i = lane; i < (16 - QPG) * 32; i += 64) reinterpret_cast<uint32_t*>(qs + QPG * 64)[i] = 0u;
  } else if (nc > 0) {
    store_round(min(nc, GQ_VRK), CptKey{}, GQ_KT);
  }
  lds_barrier();
  stamp(p, slot);
  float mrun = -INFINITY, lrun = 0.0f;
  fl_f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = fl_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const uint16_t* qrow = qs + r * 64 + c * 8;
  // value columns past the round's keys up to the chunk edge must be finite (p = 0 there)
  auto zero_tail = [&](int nr) {
    for (int i = tid; i < 64 * 16; i += NT) {
      const int col = nr + (i & 15);
      if (col < ((nr + 15) & ~15)) vt[(i >> 4) * GQ_VT_LD + col] = 0;
    }
  };
  auto put_new = [&](int t) {  // the new key into row / column t
    for (int i = tid; i < 64; i += NT) {
      ks[t * 64 + i] = kn[i];
      vt[i * GQ_VT_LD + t] = vn[i];
    }
  };
  int kb = 0, ncr = min(GQ_VRK, nc);
  const bool fits = nc < GQ_VRK;  // the new key fits the (only) round of cached keys
  bool new_in = last && fits, new_done = !last || fits;
  if (new_in) put_new(ncr);
  zero_tail(ncr + (new_in ? 1 : 0));
  lds_barrier();
  for (;;) {
    const int nr = ncr + (new_in ? 1 : 0);
    if (nr > 0) {
      const uint4 qa = *reinterpret_cast<const uint4*>(qrow);
      const uint4 qb = *reinterpret_cast<const uint4*>(qrow + 32);
      for (int ch = wave; ch * 16 < nr; ch += NWAVE) {
        const uint16_t* krow = ks + (ch * 16 + r) * 64 + c * 8;
        fl_f32x4 st = {0.0f, 0.0f, 0.0f, 0.0f};
        st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(fl_bf16x8, *reinterpret_cast<const uint4*>(krow)),
            __builtin_bit_cast(fl_bf16x8, qa), st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(fl_bf16x8, *reinterpret_cast<const uint4*>(krow + 32)),
            __builtin_bit_cast(fl_bf16x8, qb), st, 0, 0, 0);
        // st[i]: score of head row r, round key ch * 16 + 4c + i
        float sv[4], mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kl = ch * 16 + 4 * c + i;
          sv[i] = kl < nr ? st[i] * p.attn_scale * 1.4426950408889634f : -INFINITY;
          mx = fmaxf(mx, sv[i]);
        }
        mx = xor32_max(xor16_max(mx));
        const float mn = fmaxf(mrun, mx);
        const float mu = (mn == -INFINITY) ? 0.0f : mn;
        const float corr = __builtin_amdgcn_exp2f(mrun - mu);
        float pv[4];
        float ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pv[i] = __builtin_amdgcn_exp2f(sv[i] - mu);
          ps += pv[i];
        }
        ps = xor32_sum(xor16_sum(ps));
        lrun = lrun * corr + ps;
        mrun = mn;
        uint32_t ph[2], pm[2], pl[2];  // p = hi + mid + lo, three bf16 terms
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float a0 = pv[2 * e], a1 = pv[2 * e + 1];
          ph[e] = pack_bf16x2(a0, a1);
          const float r0 = a0 - bflo(ph[e]), r1 = a1 - bfhi(ph[e]);
          pm[e] = pack_bf16x2(r0, r1);
          pl[e] = pack_bf16x2(r0 - bflo(pm[e]), r1 - bfhi(pm[e]));
        }
        typedef short fl_s16x4 __attribute__((ext_vector_type(4)));
        const fl_s16x4 bh = __builtin_bit_cast(fl_s16x4, make_uint2(ph[0], ph[1]));
        const fl_s16x4 bm = __builtin_bit_cast(fl_s16x4, make_uint2(pm[0], pm[1]));
        const fl_s16x4 bl = __builtin_bit_cast(fl_s16x4, make_uint2(pl[0], pl[1]));
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          fl_f32x4 acc = o[dt];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] *= corr;
          const fl_s16x4 va = __builtin_bit_cast(
              fl_s16x4, *reinterpret_cast<const uint2*>(vt + (dt * 16 + r) * GQ_VT_LD + ch * 16 + 4 * c));
          acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, bh, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, bm, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, bl, acc, 0, 0, 0);
          o[dt] = acc;
        }
      }
    }
    if (kb + GQ_VRK < nc) {  // the next round of cached keys
      lds_barrier();         // every wave is done with this one
      kb += GQ_VRK;
      ncr = min(GQ_VRK, nc - kb);
      load_round(kb, ncr);
      new_in = last && kb + GQ_VRK >= nc && ncr < GQ_VRK;  // the last round takes the new key if it fits
      if (new_in) {
        put_new(ncr);
        new_done = true;
      }
      zero_tail(ncr + (new_in ? 1 : 0));
      lds_barrier();
    } else if (!new_done) {  // the new key in a round of its own (row 0)
      lds_barrier();
      ncr = 0;
      put_new(0);
      new_in = new_done = true;
      zero_tail(1);
      lds_barrier();
    } else {
      break;
    }
  }
  stamp(p, slot);
  // the waves' (max, sum, o) per head row: o[dt][i] at lane (r, c) is head row r, dim 16 dt + 4c + i
  if (r < GQ_ROWS) {
    float* w = wp + (wave * GQ_ROWS + r) * 66;
    if (c == 0) {
      w[0] = mrun;
      w[1] = lrun;
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) w[2 + dt * 16 + 4 * c + i] = o[dt][i];
  }
  lds_barrier();
  auto unit_word = [&](int j, int wd) {  // the unit's word wd of head row j, waves in order
    float xm[NWAVE], xv[NWAVE];  // every wave's pair read before any is used
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      xm[w] = wp[(w * GQ_ROWS + j) * 66];
      xv[w] = wp[(w * GQ_ROWS + j) * 66 + wd];
    }
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) mm = fmaxf(mm, xm[w]);
    if (wd == 0) return mm;
    float val = 0.0f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const float e = (xm[w] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(xm[w] - mm);
      val += xv[w] * e;
    }
    return val;
  };
  if (nsl == 1) {
    for (int it = tid; it < QPG * 64; it += NT) {
      const int j = it >> 6, d = it & 63;
      st_coh_u32(p.attn + (g * QPG + j) * 64 + d, f2bf(unit_word(j, 2 + d) / unit_word(j, 1)) | (otag << 16));
    }
    lds_barrier();  // wp is done with: the O phase's dequantised chunks go to the same LDS
  } else {
    const unsigned long long tg = (unsigned long long)ptag << 32;
    for (int it = tid; it < QPG * 66; it += NT) {
      const int j = it / 66, wd = it - j * 66;
      st_coh_u64(p.part + ((size_t)(g * QPG + j) * MAX_SLICES + sl) * 66 + wd,
                 (unsigned long long)__float_as_uint(unit_word(j, wd)) | tg);
    }
    lds_barrier();  // as above
    gqa_merge(p, g, sl, nsl, wp, otag, ptag);
  }
  stamp(p, slot);
}

// h[r0+2j], h[r0+2j+1] += bf16(bf16(acc) * rm) (bf16), run by the lead lane of row pair j. The
// workgroup owns these rows for the whole step (O and down share the row split), so their
// current values live in registers (ha, hb) of that lane and only the tagged result is stored.
__device__ __forceinline__ void residual_pair(const DecodeParams& p, int r0, int j, float y0,
                                              float y1, uint32_t tag, float& ha, float& hb) {
  const float o0 = rbf(rbf(y0) * p.resid_mult);
  const float o1 = rbf(rbf(y1) * p.resid_mult);
  ha = rbf(ha + o0);
  hb = rbf(hb + o1);
  const uint32_t n0 = f2bf(ha) | (tag << 16), n1 = f2bf(hb) | (tag << 16);
  st_coh_u64(reinterpret_cast<unsigned long long*>(p.h + r0) + j,
             (unsigned long long)n0 | ((unsigned long long)n1 << 32));
}

// Workgroup reductions in a fixed order (wave tree, then the waves' values in wave order), so every
// workgroup computes the bit-identical result from the same inputs. red: NWAVE floats of LDS.
__device__ __forceinline__ float wg_max_fixed(float v, float* red) {
  const int tid = tid_here();
  v = wave_max(v);
  lds_barrier();
  if ((tid & 63) == 0) red[tid >> 6] = v;
  lds_barrier();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) r = fmaxf(r, red[w]);
  return r;
}
__device__ __forceinline__ float wg_sum_fixed(float v, float* red) {
  const int tid = tid_here();
  v = wave_sum(v);
  lds_barrier();
  if ((tid & 63) == 0) red[tid >> 6] = v;
  lds_barrier();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) r += red[w];
  return r;
}
__device__ __forceinline__ uint32_t wait_u32(const DecodeParams& p, const uint32_t* a, uint32_t tag) {
  auto ld = [a]() { return ld_coh_u32(a); };
  auto ok = [tag](uint32_t v) { return (v >> 16) == tag; };
  uint32_t v = ld();
  if (!ok(v)) v = spin_until(p, v, ok, ld);
  return v;
}

// Temperature / top-k sampling fused into the decode launch, after the LM head (reference
// engine/generate.py:38-55 logits_to_probs + multinomial_sample_one_no_sync, with the same steps
// and bf16 rounding points as the standalone sampler k_sample): thread t of workgroup w holds
// x = bf16(logit / T) of LM-head row r0 + t (xl: the rows' logits in LDS). The steps that need
// the whole vocabulary exchange one value per workgroup through tagged words (tags of epochs
// e .. e + 5 after the launch's layers): the maxima; for top-k, two radix passes over the
// 16-bit ordered keys (each workgroup's 256-bin histogram; bin b's total summed by workgroup
// b % G; every workgroup reads the 256 totals and selects the pivot's bin); the partial sums of
// exp(x - max) over the kept entries, read by every workgroup and summed in one fixed order.
// Returns this thread's sample key (bf16(p / q) bits << 32 | ~index; 0 for dropped entries): the
// token is the first index of the largest key over the vocabulary.
__device__ unsigned long long sample_epilogue(const DecodeParams& p, int r0, int rows, const float* xl,
                                              int* hist, int* sel, float* red) {
  const int tid = tid_here(), G = grid_here(), wg = blockIdx.x;
  const uint32_t e = p.epoch + 5u * (uint32_t)p.NL;
  unsigned long long* tot = p.sword;
  unsigned long long* wmax = p.sword + 256;
  unsigned long long* wsum = p.sword + 256 + G;
  const bool on = tid < rows;
  const int j = r0 + tid;
  const float x = on ? rbf(xl[tid] / p.samp_tdiv) : -INFINITY;  // generate.py:42
  const uint32_t key = bf_key(x);
  const float lmx = wg_max_fixed(x, red);
  if (tid == 0)
    st_coh_u64(wmax + wg, (unsigned long long)__float_as_uint(lmx) | ((unsigned long long)tag_of(e) << 32));
  uint32_t pivot = 0;
  const bool topk = p.samp_topk > 0 && p.samp_topk < p.V;
  if (topk) {  // generate.py:44-47: keys below the k-th largest drop out, ties with it stay
    int k = p.samp_topk;
    for (int pass = 0; pass < 2; ++pass) {
      const uint32_t th = tag_of(e + 1 + 2 * pass), tt = tag_of(e + 2 + 2 * pass);
      if (tid < 256) hist[tid] = 0;
      lds_barrier();
      if (on && (pass == 0 || (key >> 8) == (pivot >> 8)))
        atomicAdd(&hist[pass == 0 ? (key >> 8) : (key & 0xFFu)], 1);
      lds_barrier();
      if (tid < 256) st_coh_u32(p.shist + (size_t)wg * 256 + tid, (uint32_t)hist[tid] | (th << 16));
      // bin b's total over the workgroups (integer counts, exact in fp32: any order)
      for (int b = wg; b < 256; b += G) {
        float c = 0.0f;
        for (int u = tid; u < G; u += NT) c += (float)(wait_u32(p, p.shist + (size_t)u * 256 + b, th) & 0xFFFFu);
        c = wg_sum_fixed(c, red);
        if (tid == 0) st_coh_u64(tot + b, (unsigned long long)(uint32_t)c | ((unsigned long long)tt << 32));
      }
      lds_barrier();
      if (tid < 256) hist[tid] = (int)(uint32_t)wait_pair(p, tot + tid, tt);
      lds_barrier();
      int above = 0;
      const int bin = select_bin(hist, k, &above, sel);
      k -= above;
      pivot = pass == 0 ? ((uint32_t)bin << 8) : (pivot | (uint32_t)bin);
      lds_barrier();
    }
  }
  // the vocabulary's max (always kept), then exp(x - max) summed over the kept entries
  float gm = -INFINITY;
  for (int u = tid; u < G; u += NT) gm = fmaxf(gm, __uint_as_float((uint32_t)wait_pair(p, wmax + u, tag_of(e))));
  gm = wg_max_fixed(gm, red);
  const bool kept = on && (!topk || key >= pivot);
  const float ex = kept ? expf(x - gm) : 0.0f;
  const float ls = wg_sum_fixed(ex, red);
  const uint32_t ts = tag_of(e + 5);
  if (tid == 0) st_coh_u64(wsum + wg, (unsigned long long)__float_as_uint(ls) | ((unsigned long long)ts << 32));
  float sp = 0.0f;
  for (int u = tid; u < G; u += NT) sp += __uint_as_float((uint32_t)wait_pair(p, wsum + u, ts));
  const float sum = wg_sum_fixed(sp, red);  // the same fixed order in every workgroup
  // p = bf16(exp(x - max) / sum); the first index of the largest bf16(p / q) (generate.py:36-38)
  unsigned long long best = 0ull;
  if (kept) {
    const float pr = rbf(ex / sum);
    if (pr != 0.0f) {  // a ratio of 0 never beats the kept maximum's
      const uint32_t r = philox_x0((uint32_t)j, 0u, p.off_lo, p.off_hi, p.seed_lo, p.seed_hi);
      const double u = ((double)(r >> 8) + 0.5) * (1.0 / 16777216.0);
      const float q = rbf((float)(-log(u)));
      const float ratio = rbf(pr / q);
      best = ((unsigned long long)__float_as_uint(ratio) << 32) | (0xFFFFFFFFu - (uint32_t)j);
    }
  }
  return best;
}

// AT, the attention of this instantiation: per-head units merging their slices in the attention
// phase (0) or, from DEFER_MERGE_SLICES slices on, in the O phase (1); by KV group (2, long
// contexts, gqa_applies). One instantiation each, picked by the host per launch, so that no
// attention's code sits in another's layer loop (the layer loop of the first is 58 KB, inside the
// 64 KB instruction cache; with the deferred merge in it, 67 KB).
template <class C, int AT>
__global__ __launch_bounds__(NT, 1) void k_decode(DecodeParams pv) {
  (void)pv;  // read through params_here()
  const DecodeParams& p = params_here();
  static_assert(PD_QKV <= C::QKV && PD_O <= C::O && PD_D + C::PR_D <= C::D &&
                    C::G3 + PD_GU + C::PR_GU <= C::NPRE_GU && C::NPRE_GU <= C::GU,
                "chunk budget");
  __shared__ __align__(16) uint16_t xs[XS_SLOTS * 8];  // staged activations (slots: xslot)
  __shared__ __align__(16) float ws[WS_FLOATS];
  __shared__ __align__(16) uint4 dql[PD_MAX * 4 * NT];  // dequantised chunks (gemv_predq)
  __shared__ float red[64];
  __shared__ unsigned long long kred[NWAVE];

  const int tid = threadIdx.x, wg = blockIdx.x, G = gridDim.x;
  const int D = p.D, F = p.F, NKV = p.NKV, NH = p.NH;
  const int NQKV = (NH + 2 * NKV) * 64;
  const int pos = p.pos;
  int slot = 0;
  stamp(p, slot);
  if (p.stall && wg == 0 && tid == 0) (void)wait_u32(p, p.stall, 1u);  // forced timeout (tests)
  // the layer-0 input: bf16(embed[token] * emb_mult), or the caller's hidden state h_io as it is
  // (reference kernels/megakernel_decode.cu:204-208 takes h; chat.py:72 forms it on the host)
  const uint16_t* erow;
  float emult = p.emb_mult;
  if (p.h_io) {
    erow = p.h_io;
    emult = 1.0f;  // bf16(x * 1) = x
  } else {
    int token = *p.token_in;
    if (token < 0 || token >= p.V) {  // bad device-side token: record it, read row 0 (no fault)
      if (tid == 0 && wg == 0)
        __hip_atomic_store(p.err, (int32_t)FL_E_ARG, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      token = 0;
    }
    erow = p.w.embed + (size_t)token * D;
  }

  int r0d, rowsd;  // this workgroup's rows of every [D]-output GEMV (O, down): it owns h there
  row_range(D, wg, G, r0d, rowsd);
  // h = bf16(embed[token] * emb_mult) on the owned rows (engine/model.py:138), held in the
  // registers of the lane that leads their row pair in the O and down epilogues
  float ha = 0.0f, hb = 0.0f;
  {
    const int lgd = row_lanes_lg(rowsd);
    const int jd = tid >> (lgd + 1);
    if ((tid & ((2 << lgd) - 1)) == 0 && 2 * jd < rowsd) {
      const uint32_t e2 = reinterpret_cast<const uint32_t*>(erow + r0d)[jd];
      ha = rbf(bflo(e2) * emult);
      hb = rbf(bfhi(e2) * emult);
    }
  }

  uint4 w_qkv[C::QKV], w_o[C::O], w_gu[C::GU], w_d[C::D];
  uint32_t s_qkv[C::QKV], s_o[C::O], s_gu[C::GU], s_d[C::D];
  // chunk mappings: O and down keep each thread in one column of chunks; QKV and gate/up go by
  // rows in the instantiations that have them (C::ROWS), else by column / by stride
  const int sD = cs_stride(D), sF = cs_stride(F);
  constexpr int M_QKV = C::ROWS ? GM_ROWS : GM_COLUMN, M_GU = C::ROWS ? GM_PAIRS : GM_STRIDE;
  auto map_qkv = [&](int n) { return C::ROWS ? map_rows(D, n) : map_stride(D, n, sD); };
  auto map_gu = [&](int n) { return C::ROWS ? map_pairs(D, n) : map_stride(D, n, NT); };
  int r0, rows;
  row_range(NQKV, wg, G, r0, rows);
  gemv_load(p.w.wqkv_q, p.w.wqkv_sz, r0, rows, D, map_qkv(rows), w_qkv, s_qkv);

  for (int l = 0; l < params_here().NL; ++l) {
    const DecodeParams& p = params_here();
    const uint32_t e0 = p.epoch + 5u * (uint32_t)l;
    const uint32_t t_prev = tag_of(e0 - 1), t_qkv = tag_of(e0), t_attn = tag_of(e0 + 1),
                   t_h1 = tag_of(e0 + 2), t_act = tag_of(e0 + 3), t_h2 = tag_of(e0 + 4);
    // Each phase polls for its inputs first and only then requests the weights of the next GEMV
    // phase: vector loads complete in order, so weights requested before a poll would delay
    // the poll's result by their whole transfer; requested after it, they stream in during this
    // phase's compute.
    int r0n, rowsn;
    // ---------------- P1: RMSNorm + QKV + RoPE + KV append ----------------
    row_range(NQKV, wg, grid_here(), r0, rows);
    // the RoPE (cos, sin) pair of the row pair this lane leads in the epilogue, requested right
    // after the residual poll's first requests (in-order returns: before them it would delay the
    // poll, after the poll's finish its latency would show in the epilogue)
    const auto rope_r = buf_rsrc(p.w.rope + (size_t)pos * 64, 128u);
    const uint32_t rope_off =
        (uint32_t)(((r0 + 2 * (tid >> ((C::ROWS ? rs_lg(rows, D >> 5) : row_lanes_lg(rows)) + 1))) &
                    63) >> 1) * 4u;
    uint32_t rope_cs = 0;
    uint32_t dq_qkv[PD_QKV][4][4] = {};  // (defined on every path: see dqe below)
    if (rows > 0) {
      if (l == 0) {
        rope_cs = buf_ld32(rope_r, rope_off);
        norm_embed(erow, emult, p.w.attn_norm, D, p.eps, xs, red);
        gemv_predq_reg(w_qkv, s_qkv, dq_qkv, [](int) {});
      } else {
        norm_tagged(p, p.h, t_prev, p.w.attn_norm + (size_t)l * D, xs, red, [&](auto refresh) {
          rope_cs = buf_ld32(rope_r, rope_off);
          gemv_predq_reg(w_qkv, s_qkv, dq_qkv, [&](int i) {  // a second look before the last
            if (i == PD_QKV - 2) refresh();
          });
        });
      }
    }
    stamp(p, slot);
    row_range(D, wg, grid_here(), r0n, rowsn);
    const NextW nx_o = next_w(p.w.wo_q + (size_t)l * D * (D >> 3),
                              p.w.wo_sz + (size_t)l * D * (D >> 7), r0n, rowsn, D,
                              map_stride(D, rowsn, sD), true);
    // (a workgroup without rows only requests the O chunks)
    gemv_compute<C::QKV, C::O, C::O, PD_QKV, M_QKV>(
        w_qkv, s_qkv, [&](int i, const uint4* x4) { return dq_dot(dq_qkv[i], x4); },
        map_qkv(rows), xs, ws, nx_o, w_o, s_o, [&](int pr, float ya, float yb) {
          const int srow = r0 + 2 * pr;
          const int hh = srow >> 6, j = (srow & 63) >> 1;
          const float a = rbf(ya), b = rbf(yb);
          float oa = a, ob = b;
          if (hh < NH + NKV) {  // RoPE (engine/model.py:257-269 on NEOX pairs j, j+32)
            const uint32_t cs = rope_cs;
            const float c = bflo(cs), sn = bfhi(cs);
            oa = rbf(a * c - b * sn);
            ob = rbf(b * c + a * sn);
          }
          st_coh_u64(p.qkv + hh * 32 + j,
                     (unsigned long long)pack_bf16x2(oa, ob) | ((unsigned long long)t_qkv << 32));
          if (hh >= NH) {  // KV append for later launches (engine/model.py:89-98)
            const int g = (hh < NH + NKV) ? hh - NH : hh - NH - NKV;
            uint16_t* dst =
                ((hh < NH + NKV) ? p.kc : p.vc) + ((size_t)(l * NKV + g) * p.S + pos) * 64;
            dst[j] = (uint16_t)f2bf(oa);
            dst[j + 32] = (uint16_t)f2bf(ob);
          }
        });
    stamp(p, slot);

    // ---------------- P2: GQA flash-decode attention ----------------
    SliceMerge mg;  // (stays empty unless AT == 1: no merge deferred to the O phase)
    if constexpr (AT == 2) {
      static_assert(C::ROWS, "the large budget's registers have no room for the attention by KV group");
      attention_gqa(p, l, t_qkv, t_attn, e0 + 1u, ws, reinterpret_cast<unsigned char*>(dql), slot);
    } else {
      attention_phase<AT == 1>(p, l, t_qkv, t_attn, e0 + 1u, ws, slot, mg);
    }
    stamp(p, slot);
    auto finish_merge = [&] {  // a deferred slice merge (wave 0, raised priority)
      if (mg.pend && tid < 64) {
        __builtin_amdgcn_s_setprio(1);
        slice_merge(p, mg, t_attn, e0 + 1u);
        __builtin_amdgcn_s_setprio(0);
      }
    };

    // ---------------- P3: O projection + residual ----------------
    row_range(D, wg, grid_here(), r0, rows);
    row_range(2 * F, wg, grid_here(), r0n, rowsn);
    const NextW nx_gu = next_w(p.w.wgu_q + (size_t)l * 2 * F * (D >> 3),
                               p.w.wgu_sz + (size_t)l * 2 * F * (D >> 7), r0n, rowsn, D,
                               map_gu(rowsn), true);
    // The wait for the attention output lasts as long as the attention chain: besides O's chunks,
    // the first G3 gate/up chunks are requested and dequantised into registers meanwhile. (The
    // arrays are defined on every path: a conditionally written array keeps its registers live
    // across the whole layer loop.)
    constexpr int G3 = C::G3 > 0 ? C::G3 : 1;
    uint32_t dqe[G3][4][4] = {};
    auto early_gu = [&] {
      if constexpr (C::G3 > 0) {
        next_load_range<0, C::G3>(nx_gu, w_gu, s_gu);
        gemv_predq_reg<C::GU, C::G3, 0>(w_gu, s_gu, dqe, [](int) {});
      }
    };
    if (rows > 0) {
      stage_tagged<POLL_D>(p, p.attn, D, t_attn, xs, [&](auto refresh) {
        if (mg.pend) {  // this workgroup's O chunks first, then the merge, then the gate/up chunks
          gemv_predq<C::O, PD_O>(w_o, s_o, dql, [&](int i) {});
          finish_merge();
          if constexpr (C::G3 > 0) next_load_range<0, C::G3>(nx_gu, w_gu, s_gu);
          refresh();
        } else {
          if constexpr (C::G3 > 0) next_load_range<0, C::G3>(nx_gu, w_gu, s_gu);
          gemv_predq<C::O, PD_O>(w_o, s_o, dql, [&](int i) {
            if (i == PD_O - 1) refresh();
          });
        }
        if constexpr (C::G3 > 0) gemv_predq_reg<C::GU, C::G3, 0>(w_gu, s_gu, dqe, [](int) {});
      });
    } else {
      finish_merge();
      early_gu();
    }
    stamp(p, slot);
    // more gate/up chunks stream in during this short phase, the rest once P4's input has
    // arrived (their transfer would otherwise delay P4's poll, which returns in order)
    gemv_compute<C::O, C::GU, C::NPRE_GU, PD_O, GM_COLUMN, C::G3>(
        w_o, s_o, [&](int i, const uint4* x4) { return dql_dot(dql, i, x4); },
        map_stride(D, rows, sD), xs,
        ws, nx_gu, w_gu, s_gu, [&](int pr, float ya, float yb) {
          residual_pair(p, r0, pr, ya, yb, t_h1, ha, hb);  // engine/model.py:162
        });
    stamp(p, slot);

    // ---------------- P4: RMSNorm + gate/up + SwiGLU ----------------
    row_range(2 * F, wg, grid_here(), r0, rows);
    constexpr int PR_GU = C::PR_GU > 0 ? C::PR_GU : 1;
    uint32_t dqr_gu[PR_GU][4][4] = {};
    if (rows > 0)
      norm_tagged(p, p.h, t_h1, p.w.ffn_norm + (size_t)l * D, xs, red, [&](auto refresh) {
        static_assert(C::PR_GU <= 1, "the second look sits in the LDS pre-dequantisation");
        gemv_predq<C::GU, PD_GU, C::G3>(w_gu, s_gu, dql, [&](int i) {  // a second look before the last
          if (i == PD_GU + C::PR_GU - 2) refresh();
        });
        if constexpr (C::PR_GU > 0)
          gemv_predq_reg<C::GU, PR_GU, C::G3 + PD_GU>(w_gu, s_gu, dqr_gu, [](int) {});
      });
    next_load_from<C::NPRE_GU>(nx_gu, w_gu, s_gu);
    stamp(p, slot);
    row_range(D, wg, grid_here(), r0n, rowsn);
    const NextW nx_d = next_w(p.w.wd_q + (size_t)l * D * (F >> 3),
                              p.w.wd_sz + (size_t)l * D * (F >> 7), r0n, rowsn, F,
                              map_stride(F, rowsn, sF), true);
    gemv_compute<C::GU, C::D, C::D, C::G3 + PD_GU + C::PR_GU, M_GU>(
        w_gu, s_gu,
        [&](int i, const uint4* x4) {  // chunks [0, G3) in dqe, then PD_GU in dql, then dqr_gu
          if (i < C::G3) return dq_dot(dqe[i < C::G3 ? i : 0], x4);
          const int k = i - C::G3;
          return k < PD_GU ? dql_dot(dql, k, x4) : dq_dot(dqr_gu[k >= PD_GU ? k - PD_GU : 0], x4);
        },
        map_gu(rows), xs, ws, nx_d, w_d, s_d, [&](int pr, float yg, float yu) {
          // act = bf16(bf16(silu(g)) * u)  (engine/model.py:227-228)
          const float g = rbf(yg), u = rbf(yu);
          st_coh_u32(p.act + (r0 >> 1) + pr, f2bf(rbf(silu_f(g)) * u) | (t_act << 16));
        });
    stamp(p, slot);

    // ---------------- P5: down projection + residual ----------------
    row_range(D, wg, grid_here(), r0, rows);
    constexpr int PR_D = C::PR_D > 0 ? C::PR_D : 1;
    uint32_t dqr_d[PR_D][4][4] = {};
    if (rows > 0)
      stage_tagged<POLL_MAX>(p, p.act, F, t_act, xs, [&](auto refresh) {
        // a second look at act before the last pre-dequantised chunk
        gemv_predq<C::D, PD_D>(w_d, s_d, dql, [&](int i) {
          if (i == PD_D + C::PR_D - 2) refresh();
        });
        if constexpr (C::PR_D > 0)
          gemv_predq_reg<C::D, PR_D, PD_D>(w_d, s_d, dqr_d, [&](int i) {
            if (i == C::PR_D - 2) refresh();
          });
      });
    stamp(p, slot);
    row_range(NQKV, wg, grid_here(), r0n, rowsn);
    const int ln = l + 1 < p.NL ? l + 1 : l;  // the last layer requests nothing
    const NextW nx_qkv = next_w(p.w.wqkv_q + (size_t)ln * NQKV * (D >> 3),
                                p.w.wqkv_sz + (size_t)ln * NQKV * (D >> 7), r0n, rowsn, D,
                                map_qkv(rowsn), l + 1 < p.NL);
    gemv_compute<C::D, C::QKV, C::QKV, PD_D + C::PR_D, GM_COLUMN>(
        w_d, s_d,
        [&](int i, const uint4* x4) {
          return i < PD_D ? dql_dot(dql, i, x4) : dq_dot(dqr_d[i >= PD_D ? i - PD_D : 0], x4);
        },
        map_stride(F, rows, sF), xs, ws, nx_qkv, w_qkv, s_qkv, [&](int pr, float ya, float yb) {
          residual_pair(p, r0, pr, ya, yb, t_h2, ha, hb);  // engine/model.py:163
        });
    stamp(p, slot);
  }
  // the final residual back into the caller's hidden state (reference decode_mega mutates h in
  // place). Every workgroup read h_io in layer 0 before its outputs could reach anyone's last
  // layer (each phase waits for every producer of the one before), so no reader remains.
  if (p.h_io) {
    const int lgd = row_lanes_lg(rowsd);
    const int jd = tid >> (lgd + 1);
    if ((tid & ((2 << lgd) - 1)) == 0 && 2 * jd < rowsd)
      reinterpret_cast<uint32_t*>(p.h_io + r0d)[jd] = pack_bf16x2(ha, hb);
  }

  // ---------------- final norm + tied bf16 LM head + greedy argmax ----------------
  const int lane = tid & 63, wave = tid >> 6;
  row_range(p.V, wg, G, r0, rows);
  const int nck = D >> 3;  // 16-byte chunks per row
  constexpr int STEP = NWAVE * LM_RB;
  uint4 ea[LM_RB][LM_MAXC], eb[LM_RB][LM_MAXC];
  unsigned long long best = 0ull;
  const auto eb_r = buf_rsrc(p.w.embed + (size_t)r0 * D, (uint32_t)rows * (uint32_t)D * 2u);
  auto lm_load = [&](uint4 (&ev)[LM_RB][LM_MAXC], int rb) {  // rows past `rows` read as 0
#pragma unroll
    for (int rr = 0; rr < LM_RB; ++rr) {
#pragma unroll
      for (int i = 0; i < LM_MAXC; ++i) {
        const int c = lane + 64 * i;
        const uint32_t off = (c < nck) ? (uint32_t)((rb + rr) * D + c * 8) * 2u : 0xFFFFFFF0u;
        ev[rr][i] = buf_ld128(eb_r, off);
      }
    }
  };
  auto lm_compute = [&](const uint4 (&ev)[LM_RB][LM_MAXC], int rb) {
#pragma unroll
    for (int rr = 0; rr < LM_RB; ++rr) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < LM_MAXC; ++i) {
        const int c = lane + 64 * i;
        if (c < nck) {
          const uint4 xv = reinterpret_cast<const uint4*>(xs)[xslot(c)];
          acc = dot2_bf16(ev[rr][i].x, xv.x, acc);
          acc = dot2_bf16(ev[rr][i].y, xv.y, acc);
          acc = dot2_bf16(ev[rr][i].z, xv.z, acc);
          acc = dot2_bf16(ev[rr][i].w, xv.w, acc);
        }
      }
      acc = wave_sum(acc);  // all-reduce: every lane holds the row's dot
      if (rb + rr < rows) {
        const int r = r0 + rb + rr;
        // logits = bf16(bf16(x . E^T) / logits_scaling)  (engine/model.py:144)
        const float lg = rbf(rbf(acc) / p.logits_scaling);
        if (p.logits && lane == 0) p.logits[r] = lg;
        if (p.samp_tdiv > 0.0f && lane == 0) ws[rb + rr] = lg;  // the rows' logits for sampling
        best = u64max(best, amax_key(lg, (uint32_t)r));
      }
    }
  };
  const int rb0 = wave * LM_RB;
  if (rb0 < rows) lm_load(ea, rb0);  // first batch in flight while the final residual arrives
  norm_tagged(p, p.h, tag_of(p.epoch + 5u * (uint32_t)p.NL - 1u), p.w.final_norm, xs, red);
  stamp(p, slot);
  if (p.feat && wg == 0)
    for (int i = tid; i < D; i += NT) p.feat[i] = xs[8 * xslot(i >> 3) + (i & 7)];
  for (int rb = rb0; rb < rows; rb += 2 * STEP) {
    if (rb + STEP < rows) lm_load(eb, rb + STEP);
    lm_compute(ea, rb);
    if (rb + 2 * STEP < rows) lm_load(ea, rb + 2 * STEP);
    if (rb + STEP < rows) lm_compute(eb, rb + STEP);
  }
  if (p.samp_tdiv > 0.0f) {  // the sampled token instead of the greedy argmax
    lds_barrier();             // the rows' logits are in ws
    int* shl = reinterpret_cast<int*>(ws + WS_FLOATS - 512);
    best = sample_epilogue(p, r0, rows, ws, shl, shl + 256, red);
    best = wave_max_u64(best);
  }
  if (lane == 0) kred[wave] = best;
  lds_barrier();
  stamp(p, slot);
  if (tid == 0) {
    unsigned long long b = kred[0];
    for (int w = 1; w < NWAVE; ++w) b = u64max(b, kred[w]);
    __hip_atomic_fetch_max(p.amax, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_mem();
    const uint32_t old = __hip_atomic_fetch_add(p.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (uint32_t)(G - 1)) {
      const unsigned long long fin = ld_coh_u64(p.amax);
      if (p.token_out) *p.token_out = (int32_t)amax_index(fin);
      __hip_atomic_store(p.amax, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ================================ speculative verify ==================================
// M <= 32 tokens through all layers in one persistent launch (reference kernels/verify_mega.cu:
// 106-283 verify_mega<M>, M in {1..16, 20, 24, 28, 32}): token m sits at cache slot pos+m, takes
// RoPE position pos+depth[m] and attends to the cache [0, pos) plus the new tokens j with
// amask[m][j] != 0. Five phases per layer as k_decode. Every GEMM runs on the matrix cores: a
// workgroup takes 16-row weight tiles, its 8 waves split the K groups, each lane dequantises one
// 16-byte chunk per group and feeds four v_mfma_f32_16x16x32_bf16 steps against up to 16 token
// rows staged in LDS (rows past the pass's tokens read a zero row); more than 16 tokens take two
// passes over the phase's tiles. The tied LM head is an MFMA tile over the bf16 embedding.
//
// The vectors every workgroup stages (the residual h before the two RMSNorms and the LM head, the
// attention output before the O projection, a K part of the SwiGLU output before the down
// projection) go through plain bf16 buffers with one ready flag per producing block (a weight
// tile, an attention unit): a producer stores its values, waits until they are written
// (s_waitcnt) and only then stores its flag (the phase's tag); a consumer polls the flags of the
// blocks it needs, then copies the rows. That is half the bytes of one tagged 32-bit word per
// value, and those bytes bound these hand-offs: every workgroup reads the same M rows (about
// 4 TB/s summed over the chip for these reads). q / k / v and the down projection's part sums
// stay tagged words. Each workgroup keeps its own 16 rows of the residual in LDS for the whole
// launch, as k_decode keeps them in registers.
constexpr int VH = 16;  // token rows per pass through a GEMM phase (one MFMA row block)
constexpr int VT_NB = 8;  // tiles per batch of the tile dequantisation steps (unit_mma_t)

// Verify attention (see attention_verify): keys per load round VRK; LDS regions of a unit, in
// bytes from the region's start.
constexpr int VRK = 256;
constexpr int VT_LD = VRK + 8;  // V^T row pitch (bf16)
constexpr int VA_Q = 0;                                   // q rows [32][64] bf16
constexpr int VA_K = VA_Q + FL_MAX_VERIFY * 128;          // key rows [VRK][64] bf16
constexpr int VA_VT = VA_K + VRK * 128;                   // values, transposed [64][VT_LD] bf16
constexpr int VA_MASK = VA_VT + 64 * VT_LD * 2;           // tree mask rows [32][32] u8
constexpr int VA_WP = VA_MASK + FL_MAX_VERIFY * FL_MAX_VERIFY;  // per-wave partials [NWAVE][16][66] fp32
constexpr int VA_BYTES = VA_WP + NWAVE * 16 * 66 * 4;

// dynamic LDS of k_verify: a region shared by the staged token rows of the GEMM phases
// ([VH + 1][D + 8] bf16, row VH stays zero) and the attention unit (VA_BYTES), the current
// RMSNorm weight vector as two masked copies (stage_norm_w: 2 x [D] bf16), per-wave tile partials
// [4][8][256] floats and this workgroup's rows of the residual h [32][16] (bf16)
__host__ __device__ inline size_t verify_xs_bytes(int D) {
  const size_t xs = ((size_t)(VH + 1) * (D + 8) * 2 + 15) & ~(size_t)15;
  return xs > (size_t)VA_BYTES ? xs : (size_t)VA_BYTES;
}
__host__ __device__ inline size_t verify_nw_bytes(int D) { return ((size_t)D * 4 + 15) & ~(size_t)15; }
constexpr int VPART_TILES = 5;  // tiles whose wave partials the LDS holds at once (down projection rounds)
inline size_t verify_lds_bytes(int D) {
  return verify_xs_bytes(D) + verify_nw_bytes(D) + VPART_TILES * NWAVE * 256 * 4 + FL_MAX_VERIFY * 16 * 2;
}

// A norm weight vector (bf16 [D], D % 8 == 0) into LDS as two copies of its bf16 pairs, one with
// the high half cleared (w_2k, 0) and one with the low half cleared (0, w_2k+1): a v_dot2 of a
// packed pair with them is the one product x_2k * w_2k (or x_2k+1 * w_2k+1), exact in fp32, with
// no unpacking (norm_rows). Called before a phase's input wait: its loads complete while the
// workgroup waits, so the norm after the wait reads no global memory (a global load there would
// queue behind the weight tiles requested before the wait and wait for all of them: loads
// complete in order).
__device__ __forceinline__ void stage_norm_w(const uint16_t* __restrict__ nw, int D, uint16_t* nws) {
  uint4* const lo = reinterpret_cast<uint4*>(nws);
  uint4* const hi = lo + (D >> 3);
  for (int i = tid_here(); i < (D >> 3); i += NT) {
    const uint4 w = reinterpret_cast<const uint4*>(nw)[i];
    lo[i] = make_uint4(w.x & 0xFFFFu, w.y & 0xFFFFu, w.z & 0xFFFFu, w.w & 0xFFFFu);
    hi[i] = make_uint4(w.x & 0xFFFF0000u, w.y & 0xFFFF0000u, w.z & 0xFFFF0000u, w.w & 0xFFFF0000u);
  }
}

// verify's ready flags (uint32 words, tag << 16): per O tile (h1), per down tile (h2), per query
// head (attention output), per gate/up tile (SwiGLU output)
constexpr int VF_H1 = 0, VF_H2 = 256, VF_ATTN = 512, VF_ACT = VF_ATTN + 256;
constexpr int VF_WORDS = VF_ACT + 2048;

// Key slices of verify attention per query head: nsl units, one per p.vkps cached keys (default 128)
// but at most VNS, G / NH (so all units of a launch fit the grid, one each) and
// (VF_ACT - VF_ATTN) / NH (each unit's ready flag VF_ATTN + head * nsl + s stays inside the
// attention flag region on any grid; the host accepts NH <= VF_ACT - VF_ATTN), unit s covering the
// cached keys [s kps, min(pos, (s+1) kps)) (kps a multiple of 16); the last unit also takes the
// new keys. With pos <= p.vkps there is one unit per head and no merge.
constexpr int VNS = 16;
__device__ __forceinline__ void verify_slices(const DecodeParams& p, int pos, int NH, int G, int& nsl, int& kps) {
  const int ch = (pos + 15) >> 4;
  const int cap = max(1, min(min(VNS, G / NH), (VF_ACT - VF_ATTN) / NH));
  nsl = max(1, min(cap, (pos + p.vkps - 1) / p.vkps));  // a slice per vkps keys, while units last
  kps = ((ch + nsl - 1) / nsl) * 16;
  nsl = kps ? max(1, (pos + kps - 1) / kps) : 1;
}

// Ready flags order the bf16 rows without fences (which on gfx950 write back / invalidate a whole
// L2): rows are stored with agent-scope stores (sc1, written through to the coherence point) and
// read with agent-scope loads (sc1, never served from a non-coherent cached copy). A producer
// waits until all its stores are complete (s_waitcnt 0) before one thread stores the flag, and a
// consumer issues its row loads only after the flag loads have returned the tag, so the rows it
// reads are the ones written before the flag. The empty asm statements keep the compiler from
// moving memory accesses across the hand-off.
__device__ __forceinline__ void wait_flags(const DecodeParams& p, const uint32_t* flags, int n, uint32_t tag) {
  // wave 0 polls the flags four to a lane, one 16-byte load per lane per poll (flags 16-byte
  // aligned): a workgroup that waits puts at most 64 loads per poll on the flags' few memory
  // lines instead of one per flag and thread
  if (tid_here() < 64) {
    const int lane = tid_here();
    for (int b = 0; b < n; b += 256) {
      const auto rs = buf_rsrc(flags + b, (uint32_t)min(256, n - b) * 4u);
      auto mine_ok = [&](uint4 v) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        bool ok = true;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (b + 4 * lane + e < n && (w[e] >> 16) != tag) ok = false;
        return ok;
      };
      uint4 v = buf_ld128_coh(rs, (uint32_t)lane * 16u);
      unsigned long long t0 = 0;
      for (unsigned it = 0;; ++it) {
        const bool ok = mine_ok(v);
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
        if (it == 0) t0 = __builtin_amdgcn_s_memrealtime();
        __builtin_amdgcn_s_sleep(2);
        if (!ok) v = buf_ld128_coh(rs, (uint32_t)lane * 16u);
        if (__builtin_expect((it & 63u) == 63u, 0)) {
          if (__hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
          if (__builtin_amdgcn_s_memrealtime() - t0 > p.spin_ticks) {
            __hip_atomic_store(p.err, (int32_t)FL_E_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
        }
      }
    }
  }
  asm volatile("" ::: "memory");
  lds_barrier();
  asm volatile("" ::: "memory");
}
// The workgroup's rows are written: every thread waits until its own stores are complete.
__device__ __forceinline__ void release_rows() {
  asm volatile("" ::: "memory");
  wait_mem();
  lds_barrier();
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ void set_flag(uint32_t* flag, uint32_t tag) {
  release_rows();
  if (tid_here() == 0) st_coh_u32(flag, tag << 16);
}

// Rows m0 .. m0+mh-1 of a bf16 [*, stride] buffer, columns k0 .. k0+kn-1 (kn % 8 == 0), into xs
// rows 0 .. mh-1 (row pitch ld): 16-byte device-coherent loads, up to SB per thread in flight.
__device__ void stage_bf16(const uint16_t* src, int stride, int m0, int mh, int k0, int kn,
                           uint16_t* xs, int ld) {
  constexpr int SB = 8;
  const int tid = tid_here();
  const int cpr = kn >> 3, total = mh * cpr;
  const auto rsrc = buf_rsrc(src, (uint32_t)(m0 + mh) * (uint32_t)stride * 2u);
  for (int base = 0; base < total; base += SB * NT) {
    uint4 v[SB];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const int idx = base + tid + i * NT;
      const int m = idx / cpr, c = idx - m * cpr;
      v[i] = buf_ld128_coh(rsrc, idx < total ? (uint32_t)(((m0 + m) * stride + k0 + 8 * c) * 2) : 0xFFFFFFF0u);
    }
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const int idx = base + tid + i * NT;
      if (idx < total) {
        const int m = idx / cpr, c = idx - m * cpr;
        *reinterpret_cast<uint4*>(xs + m * ld + 8 * c) = v[i];
      }
    }
  }
}

// rows m < M of xs: x <- bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)  (engine/model.py:237-242).
// A row is shared by NWAVE / M waves (all 8 for one token), whose partial sums of squares meet
// in red (NWAVE floats of LDS); the row loop has the same trip count in every wave, so the
// barriers are uniform. A lane's chunks are read four at a time (independent LDS reads in flight
// instead of one round trip per chunk); nw is the weight vector in LDS as stage_norm_w leaves it.
// The squares are summed two per v_dot2 (fp32, in a different order than torch's reduction);
// x * r is an fp32 multiply, rounded to bf16 by v_cvt_pk_bf16_f32, and its product with w one
// v_dot2 against the masked weight pair (the bf16 product is exact in fp32, so the result is the
// reference's bf16(bf16(x * r) * w); an exact zero product may come out as +0 where torch gives -0).
__device__ __forceinline__ void norm_rows(uint16_t* xs, int ld, int M, int D, const uint16_t* nw,
                                          float eps, float* red) {
  constexpr int CB = 4;  // chunks per batch
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  int wpr = 1;                                  // waves per row: a power of two, wpr * M <= NWAVE
  while (wpr * 2 * M <= NWAVE) wpr *= 2;
  const int rpp = NWAVE / wpr;                  // rows per pass
  const int sub = wave % wpr, nch = D >> 3;     // this wave's share of a row; 8-value chunks per row
  const int step = wpr * 64;                    // chunk stride of a lane
  const uint4* const nwlo = reinterpret_cast<const uint4*>(nw);
  const uint4* const nwhi = nwlo + nch;
  for (int m0 = 0; m0 < M; m0 += rpp) {
    const int m = m0 + wave / wpr;
    const bool on = m < M;
    uint4* row = reinterpret_cast<uint4*>(xs + (on ? m : 0) * ld);
    float ss = 0.0f;
    for (int c0 = sub * 64 + lane; c0 < nch; c0 += CB * step) {
      uint4 v[CB];
#pragma unroll
      for (int b = 0; b < CB; ++b) {
        const int i = c0 + b * step;
        v[b] = (on && i < nch) ? row[i] : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int b = 0; b < CB; ++b) {
        const uint32_t in[4] = {v[b].x, v[b].y, v[b].z, v[b].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) ss = dot2_bf16(in[j], in[j], ss);
      }
    }
    ss = wave_sum(ss);
    if (wpr > 1) {
      if (lane == 0) red[wave] = ss;
      lds_barrier();
      ss = 0.0f;
      for (int w = 0; w < wpr; ++w) ss += red[(wave / wpr) * wpr + w];
    }
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
    if (on)
      for (int c0 = sub * 64 + lane; c0 < nch; c0 += CB * step) {
        uint4 v[CB], gl[CB], gh[CB];
#pragma unroll
        for (int b = 0; b < CB; ++b) {
          const int i = min(c0 + b * step, nch - 1);
          v[b] = row[i];
          gl[b] = nwlo[i];
          gh[b] = nwhi[i];
        }
#pragma unroll
        for (int b = 0; b < CB; ++b) {
          if (c0 + b * step < nch) {
            const uint32_t in[4] = {v[b].x, v[b].y, v[b].z, v[b].w};
            const uint32_t wl[4] = {gl[b].x, gl[b].y, gl[b].z, gl[b].w};
            const uint32_t wh[4] = {gh[b].x, gh[b].y, gh[b].z, gh[b].w};
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t n2 = pack_bf16x2(bflo(in[j]) * r, bfhi(in[j]) * r);  // bf16(x * r) pair
              o[j] = pack_bf16x2(dot2_bf16(n2, wl[j], -0.0f), dot2_bf16(n2, wh[j], -0.0f));
            }
            row[c0 + b * step] = make_uint4(o[0], o[1], o[2], o[3]);
          }
        }
      }
    if (wpr > 1) lds_barrier();  // red is reused by the next pass
  }
}

// norm_rows of rows m0 .. m0+mh-1 of the bf16 [*, D] buffer src into xs rows 0 .. mh-1, fused with
// their staging: each wave loads its share of a row (the chunks norm_rows gives it) with 16-byte
// device-coherent loads straight into registers, sums the squares there and writes only the
// normalised values to LDS. The same arithmetic in the same order as stage_bf16 + norm_rows, with
// one LDS write per chunk instead of a staging write, two row reads and a write (at M = 8 the
// separate norm took 2.1 us of a workgroup's time per phase, measured with in-kernel
// timestamps). Ends with a barrier.
__device__ __forceinline__ void stage_norm_rows(const uint16_t* src, int m0, int mh, int D, uint16_t* xs,
                                                int ld, const uint16_t* nw, float eps, float* red) {
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  int wpr = 1;  // waves per row, as norm_rows
  while (wpr * 2 * mh <= NWAVE) wpr *= 2;
  const int rpp = NWAVE / wpr, sub = wave % wpr, nch = D >> 3, step = wpr * 64;
  const auto rs = buf_rsrc(src + (size_t)m0 * D, (uint32_t)mh * (uint32_t)D * 2u);
  const uint4* const nwlo = reinterpret_cast<const uint4*>(nw);
  const uint4* const nwhi = nwlo + nch;
  for (int r0 = 0; r0 < mh; r0 += rpp) {
    const int m = r0 + wave / wpr;
    const bool on = m < mh;
    uint4 v[LM_MAXC];  // D <= 64 * 8 * LM_MAXC
#pragma unroll
    for (int j = 0; j < LM_MAXC; ++j) {  // chunks past the row read as 0, touching no memory
      const int c = sub * 64 + lane + j * step;
      v[j] = buf_ld128_coh(rs, (on && c < nch) ? (uint32_t)(m * D + c * 8) * 2u : 0xFFFFFFF0u);
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < LM_MAXC; ++j) {
      const uint32_t in[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) ss = dot2_bf16(in[e], in[e], ss);
    }
    ss = wave_sum(ss);
    if (wpr > 1) {
      if (lane == 0) red[wave] = ss;
      lds_barrier();
      ss = 0.0f;
      for (int w = 0; w < wpr; ++w) ss += red[(wave / wpr) * wpr + w];
    }
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
    uint4* const row = reinterpret_cast<uint4*>(xs + (on ? m : 0) * ld);
#pragma unroll
    for (int j = 0; j < LM_MAXC; ++j) {
      const int c = sub * 64 + lane + j * step;
      if (on && c < nch) {
        const uint4 gl = nwlo[c], gh = nwhi[c];
        const uint32_t in[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        const uint32_t wl[4] = {gl.x, gl.y, gl.z, gl.w};
        const uint32_t wh[4] = {gh.x, gh.y, gh.z, gh.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t n2 = pack_bf16x2(bflo(in[e]) * r, bfhi(in[e]) * r);  // bf16(x * r) pair
          o[e] = pack_bf16x2(dot2_bf16(n2, wl[e], -0.0f), dot2_bf16(n2, wh[e], -0.0f));
        }
        row[c] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
    if (wpr > 1) lds_barrier();  // red is reused by the next pass
  }
  lds_barrier();
}

// The weights of one 16-row tile of an [N, K] int4 matrix in the tiled layout (fl_tile_int4:
// 1 KB per 16 rows x 128-group unit, 16 bytes per lane) over the K groups g0 .. g0+ng-1
// (ng <= NWAVE * TW_G): this wave's groups g0 + wave + 8i, one unit each. rows = 16, or 0 to
// request nothing (every load past the range reads zeros). Loading does not depend on the token
// rows, so QKV and gate/up request tiles before they wait for their inputs, and every phase
// requests the next tile before it computes the current one. Loads complete in order: rows
// staged after a tile's request arrive only after that tile (measured faster all the same in
// every phase: the tiles arrive during the wait).
constexpr int TW_G = 3;  // K groups per wave of a tile: D <= 3072 is at most 24 groups, 3 per wave
static_assert(TW_G * NWAVE * 128 >= 64 * 8 * LM_MAXC, "a tile's K groups fit TW_G per wave at the largest D");
struct TileW {
  uint4 w[TW_G];
  uint32_t s[TW_G];
};
__device__ __forceinline__ void tile_load(const uint32_t* __restrict__ qt, const uint32_t* __restrict__ sz,
                                          int n0, int rows, int K, int g0, int ng, TileW& tw) {
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  const int r = lane & 15;
  const int groups = K >> 7;
  const auto wr = buf_rsrc(qt + (size_t)n0 * (K >> 3), (uint32_t)rows * (uint32_t)(K >> 1));
  const auto sr = buf_rsrc(sz + (size_t)n0 * groups, (uint32_t)rows * (uint32_t)groups * 4u);
#pragma unroll
  for (int i = 0; i < TW_G; ++i) {
    const int u = wave + NWAVE * i;
    const uint32_t gg = (uint32_t)(g0 + u);
    const bool in = u < ng;
    tw.w[i] = buf_ld128(wr, in ? (gg * 64u + (uint32_t)lane) * 16u : 0xFFFFFFF0u);
    tw.s[i] = buf_ld32(sr, in ? ((uint32_t)r * (uint32_t)groups + gg) * 4u : 0xFFFFFFF0u);
  }
}
// acc += X(token rows 0 .. mh-1 of xs) . dq(tile)^T; xs column 0 = group g0 of the tile's K range.
// Both exact dequantisation steps on 4x4x4 MFMAs, the dot on 16x16x32 MFMAs (unit_mma_t): lane L
// reads token row L % 16 (or the zero row VH) at columns 32tp + 4 (L / 16) (+ 16) of each group.
__device__ __forceinline__ void tile_mma(const TileW& tw, int ng, const uint16_t* xs, int ld, int mh,
                                         fl_f32x4& acc) {
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  const int r = lane & 15, c = lane >> 4;
  const uint16_t* xrow = xs + (r < mh ? r : VH) * ld + 4 * c;
  const MxLane m = mx_lane();
#pragma unroll
  for (int i = 0; i < TW_G; ++i) {
    const int u = wave + NWAVE * i;
    if (u < ng) unit_mma_t<VT_NB>(tw.w[i], tw.s[i], m, xrow + u * 128, acc);  // wave-uniform
  }
}

// the waves' tile partials -> part[wave][token * 16 + row]; ends with a barrier
__device__ __forceinline__ void tile_publish(float* part, const fl_f32x4& acc) {
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  const int r = lane & 15, c = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) part[wave * 256 + (c * 4 + i) * 16 + r] = acc[i];
  lds_barrier();
}
// One group per wave (group g0 + wave of a 16-row tile, waves past ng idle): the down
// projection's K parts, whose tiles are all requested at once.
struct TileW1 {
  uint4 w;
  uint32_t s;
};
__device__ __forceinline__ void tile_load1(const uint32_t* __restrict__ qt, const uint32_t* __restrict__ sz,
                                           int n0, int K, int g0, int ng, TileW1& tw) {
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  const int r = lane & 15, groups = K >> 7;
  const auto wr = buf_rsrc(qt + (size_t)n0 * (K >> 3), 16u * (uint32_t)(K >> 1));
  const auto sr = buf_rsrc(sz + (size_t)n0 * groups, 16u * (uint32_t)groups * 4u);
  const bool in = wave < ng;
  const uint32_t gg = (uint32_t)(g0 + wave);
  tw.w = buf_ld128(wr, in ? (gg * 64u + (uint32_t)lane) * 16u : 0xFFFFFFF0u);
  tw.s = buf_ld32(sr, in ? ((uint32_t)r * (uint32_t)groups + gg) * 4u : 0xFFFFFFF0u);
}
__device__ __forceinline__ void tile_mma1(const TileW1& tw, int ng, const uint16_t* xs, int ld, int mh,
                                          fl_f32x4& acc) {
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  const int r = lane & 15, c = lane >> 4;
  if (wave < ng)  // wave-uniform
    unit_mma_t<VT_NB>(tw.w, tw.s, mx_lane(), xs + (r < mh ? r : VH) * ld + wave * 128 + 4 * c, acc);
}

// The activation fragment tile_mma1 reads, from the bf16 [*, stride] rows src (device-coherent
// loads) into the same place of xs: lane (r, c) of wave w copies row m0 + r (r < mh, w < ng),
// columns k0 + 128 w + 32 tp + 4 c + 0..3 and + 16 + 0..3 (tp = 0..3), to xs row r at the same
// columns less k0. Each lane later reads back only its own fragment, so the copy needs no barrier.
__device__ __forceinline__ void stage_frag(const uint16_t* src, int stride, int m0, int mh, int k0, int ng,
                                           uint16_t* xs, int ld) {
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  const int r = lane & 15, c = lane >> 4;
  if (r >= mh || wave >= ng) return;  // rows past mh read xs row VH (zero)
  const auto rs = buf_rsrc(src + (size_t)m0 * stride, (uint32_t)mh * (uint32_t)stride * 2u);
  uint2 v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    v[e] = buf_ld64_coh(rs, (uint32_t)(r * stride + k0 + wave * 128 + 32 * (e >> 1) + 16 * (e & 1) + 4 * c) * 2u);
  uint16_t* const dst = xs + r * ld + wave * 128 + 4 * c;
#pragma unroll
  for (int e = 0; e < 8; ++e) *reinterpret_cast<uint2*>(dst + 32 * (e >> 1) + 16 * (e & 1)) = v[e];
}

// four tiles' partials at once: tile i's go to part + i * NWAVE * 256; ends with a barrier
template <int N>
__device__ __forceinline__ void tile_publish4(float* part, const fl_f32x4 (&acc)[N]) {
  const int lane = tid_here() & 63, wave = tid_here() >> 6;
  const int r = lane & 15, c = lane >> 4;
#pragma unroll
  for (int t = 0; t < N; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) part[(t * NWAVE + wave) * 256 + (c * 4 + i) * 16 + r] = acc[t][i];
  lds_barrier();
}
// sum over the waves (fixed order) of entry t = token * 16 + row
__device__ __forceinline__ float tile_sum(const float* part, int t) {
  float v = 0.0f;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) v += part[w * 256 + t];
  return v;
}

// tokens per attention unit and units per head (attention by tokens): the fewest tokens per unit
// (at most VH) that give every workgroup at most one unit, where such a count exists
__host__ __device__ inline void verify_units(int NH, int M, int G, int& tpu, int& ngrp) {
  const int t0 = (NH * M + G - 1) / G, mx = M < VH ? M : VH;
  tpu = t0 < VH ? t0 : VH;
  while (tpu < mx && NH * ((M + tpu - 1) / tpu) > G) ++tpu;
  ngrp = (M + tpu - 1) / tpu;
}

// One pass of the by-tokens attention over tokens m0 + mi0 .. m0 + mi0 + nt - 1 (nt <= TT) of
// head hq: the waves take interleaved 8-key steps over the cached keys [0, pos), RB steps per
// round of registers, each K / V step used for all TT queries (lane (kk = lane / 8, ds = lane % 8)
// holds dims 8ds..8ds+7 of key kk: q.k is 4 dot2 plus a 3-step DPP sum, p.v 8 FMAs per query);
// wave 0 folds in the new keys under the tree mask; the waves merge through LDS and the pass
// writes bf16(o / sum) of its tokens to vattn. Query slots past nt compute on token m0 + mi0 and
// are not written.
template <int TT, int RB>
__device__ __forceinline__ void attn_tokens_pass(const DecodeParams& p, int pos, int M, int m0,
                                                 int mi0, int nt, int hq, int l, int g, float sc,
                                                 const uint32_t* att32, const uint16_t* katt,
                                                 const uint16_t* vatt, const uint8_t* amk,
                                                 float* wpart) {
  const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
  const int kk = lane >> 3, ds = lane & 7;
  const int NKV = p.NKV;
  const int ns = (pos + 7) >> 3;  // 8-key steps over the cached keys [0, pos)
  const int nrounds = (ns + NWAVE * RB - 1) / (NWAVE * RB);
  const size_t cbase = (size_t)(l * NKV + g) * p.S * 64;
  const auto kb = buf_rsrc(p.kc + cbase, (uint32_t)pos * 128u);
  const auto vb = buf_rsrc(p.vc + cbase, (uint32_t)pos * 128u);
  uint4 kr[RB], vr[RB];
  auto issue = [&](int r) {
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const uint32_t off = (uint32_t)(((r * NWAVE * RB + wave + NWAVE * i) * 8 + kk) * 128 + ds * 16);
      kr[i] = buf_ld128(kb, off);
      vr[i] = buf_ld128(vb, off);
    }
  };
  if (nrounds > 0) issue(0);
  uint32_t qv[TT][4];
  float mx[TT], lsum[TT], o[TT][8];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int mi = mi0 + (t < nt ? t : 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[t][e] = att32[mi * 32 + ds * 4 + e];
    mx[t] = -INFINITY;
    lsum[t] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[t][e] = 0.0f;
  }
  for (int r = 0; r < nrounds; ++r) {
    if (r > 0) issue(r);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t >= nt) break;  // uniform: a pass with fewer tokens skips the unused query slots
      float s[RB];
      float rmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int st = r * NWAVE * RB + wave + NWAVE * i;
        float a = dot2_bf16(kr[i].x, qv[t][0], 0.0f);
        a = dot2_bf16(kr[i].y, qv[t][1], a);
        a = dot2_bf16(kr[i].z, qv[t][2], a);
        a = dot2_bf16(kr[i].w, qv[t][3], a);
        a = sum8(a);
        s[i] = (st * 8 + kk < pos) ? a * sc : -INFINITY;
        rmax = fmaxf(rmax, s[i]);
      }
      const float mn = fmaxf(mx[t], max_stride8(rmax));
      const float mu = (mn == -INFINITY) ? 0.0f : mn;
      const float corr = __builtin_amdgcn_exp2f(mx[t] - mu);
      lsum[t] *= corr;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[t][e] *= corr;
      mx[t] = mn;
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const float pw = __builtin_amdgcn_exp2f(s[i] - mu);
        lsum[t] += pw;
        o[t][0] = __builtin_fmaf(pw, bflo(vr[i].x), o[t][0]);
        o[t][1] = __builtin_fmaf(pw, bfhi(vr[i].x), o[t][1]);
        o[t][2] = __builtin_fmaf(pw, bflo(vr[i].y), o[t][2]);
        o[t][3] = __builtin_fmaf(pw, bfhi(vr[i].y), o[t][3]);
        o[t][4] = __builtin_fmaf(pw, bflo(vr[i].z), o[t][4]);
        o[t][5] = __builtin_fmaf(pw, bfhi(vr[i].z), o[t][5]);
        o[t][6] = __builtin_fmaf(pw, bflo(vr[i].w), o[t][6]);
        o[t][7] = __builtin_fmaf(pw, bfhi(vr[i].w), o[t][7]);
      }
    }
  }
  if (wave == 0) {  // the new tokens' keys, 8 per step, masked by amask[m][.]
    for (int s0 = 0; s0 < M; s0 += 8) {
      const int jn = s0 + kk;
      const int js = min(jn, M - 1);
      const uint32_t* kw = reinterpret_cast<const uint32_t*>(katt) + js * 32 + ds * 4;
      const uint32_t* vw = reinterpret_cast<const uint32_t*>(vatt) + js * 32 + ds * 4;
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t >= nt) break;
        const int mi = mi0 + t;
        const bool valid = jn < M && amk[mi * M + js] != 0;
        float a = dot2_bf16(kw[0], qv[t][0], 0.0f);
        a = dot2_bf16(kw[1], qv[t][1], a);
        a = dot2_bf16(kw[2], qv[t][2], a);
        a = dot2_bf16(kw[3], qv[t][3], a);
        a = sum8(a);
        const float sn = valid ? a * sc : -INFINITY;
        const float mn = fmaxf(mx[t], max_stride8(sn));
        const float mu = (mn == -INFINITY) ? 0.0f : mn;
        const float corr = __builtin_amdgcn_exp2f(mx[t] - mu);
        const float pw = __builtin_amdgcn_exp2f(sn - mu);
        lsum[t] = lsum[t] * corr + pw;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[t][2 * e] = __builtin_fmaf(pw, bflo(vw[e]), o[t][2 * e] * corr);
          o[t][2 * e + 1] = __builtin_fmaf(pw, bfhi(vw[e]), o[t][2 * e + 1] * corr);
        }
        mx[t] = mn;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    lsum[t] = sum_stride8(lsum[t]);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[t][e] = sum_stride8(o[t][e]);
    float* mywp = wpart + (t * NWAVE + wave) * 66;
    if (kk == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) mywp[2 + ds * 8 + e] = o[t][e];
    }
    if (lane == 0) {
      mywp[0] = mx[t];
      mywp[1] = lsum[t];
    }
  }
  lds_barrier();
  if (tid < 64 * nt) {  // thread (token t, dim d): the waves merged in a fixed order
    const int t = tid >> 6, d = tid & 63;
    const float* wt = wpart + t * NWAVE * 66;
    float M_ = -INFINITY, Ls = 0.0f, O = 0.0f;
    float wmx[NWAVE], wls[NWAVE], wov[NWAVE];  // all read before any is used, as in decode
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      wmx[w] = wt[w * 66];
      wls[w] = wt[w * 66 + 1];
      wov[w] = wt[w * 66 + 2 + d];
    }
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) M_ = fmaxf(M_, wmx[w]);
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const float e = (wmx[w] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(wmx[w] - M_);
      Ls += wls[w] * e;
      O += wov[w] * e;
    }
    st_coh_u16(p.vattn + (size_t)(m0 + mi0 + t) * p.D + hq * 64 + d, f2bf(O / Ls));
  }
  lds_barrier();
}

// Verify attention by tokens (engine/model.py:171-179 over the verify key set), for few tokens
// at short and medium contexts, where it needs no merge across workgroups. A unit is one query head and a
// group of TPU consecutive tokens (verify_units: the fewest that give every workgroup at most one
// unit); the unit runs its tokens two at a time over the head's cached keys (attn_tokens_pass),
// each key's K / V registers serving both queries. LDS att: q of the unit's tokens [VH][64], then the new k and v of the group
// [FL_MAX_VERIFY][64] each; amk: the unit's amask rows [TPU][M]. The outputs go to the bf16
// buffer vattn, then the unit's ready flag (VF_ATTN + group * NH + head).
__device__ void attention_verify_tokens(const DecodeParams& p, int l, uint32_t qtag, uint32_t otag,
                                        unsigned char* ua, int& slot) {
  uint16_t* const att = reinterpret_cast<uint16_t*>(ua);                        // q [VH][64], new k, v [32][64]
  uint8_t* const amk = ua + (VH + 2 * FL_MAX_VERIFY) * 64 * 2;                  // [VH][32]
  float* const wpart = reinterpret_cast<float*>(amk + VH * FL_MAX_VERIFY);      // [2][NWAVE][66]
  stamp(p, slot);
  stamp(p, slot);
  const int tid = tid_here();
  const int M = p.M, pos = p.pos, NH = p.NH, NKV = p.NKV, QPG = p.NH / p.NKV;
  const int HALF = (NH + 2 * NKV) * 32;  // tagged pairs per token
  int TPU, ngrp;
  verify_units(NH, M, (int)gridDim.x, TPU, ngrp);
  const float sc = p.attn_scale * 1.4426950408889634f;
  const uint32_t* att32 = reinterpret_cast<const uint32_t*>(att);
  uint16_t* const katt = att + VH * 64;                  // new k [FL_MAX_VERIFY][64]
  uint16_t* const vatt = att + (VH + FL_MAX_VERIFY) * 64;  // new v
  for (int u = blockIdx.x; u < NH * ngrp; u += gridDim.x) {
    const int g = u % NKV, rest = u / NKV, j = rest % QPG, grp = rest / QPG;
    const int hq = g * QPG + j, m0 = grp * TPU, mt = min(M, m0 + TPU) - m0;
    const int nq = 32 * mt;
    for (int i = tid; i < nq + 64 * M; i += NT) {
      int hh, tok, d;
      uint16_t* dst;
      if (i < nq) {
        hh = hq, tok = m0 + (i >> 5), d = i & 31, dst = att + (i >> 5) * 64;
      } else {
        const int i2 = i - nq, which = i2 / (32 * M), r2 = i2 - which * 32 * M;
        tok = r2 >> 5, d = r2 & 31;
        hh = which ? NH + NKV + g : NH + g;
        dst = (which ? vatt : katt) + tok * 64;
      }
      const unsigned long long v = wait_pair(p, p.qkv + (size_t)tok * HALF + hh * 32 + d, qtag);
      dst[d] = (uint16_t)v;
      dst[d + 32] = (uint16_t)(v >> 16);
    }
    for (int i = tid; i < mt * M; i += NT) amk[i] = p.amask[m0 * M + i];
    lds_barrier();
    // the unit's tokens, TT at a time: each key step's K / V registers serve all TT queries
    for (int mi0 = 0; mi0 < mt; mi0 += 2)
      attn_tokens_pass<2, 8>(p, pos, M, m0, mi0, min(2, mt - mi0), hq, l, g, sc, att32, katt, vatt, amk, wpart);
    set_flag(p.vflag + VF_ATTN + grp * NH + hq, otag);
  }
  stamp(p, slot);
  stamp(p, slot);
}

// Verify attention (engine/model.py:171-179 over the verify key set; q.k^T * scale, softmax and
// p.v in fp32, bf16 output). Token m's query attends to the cached keys [0, pos) and to the new
// keys t (this launch's tokens, from the q/k/v exchange) with amask[m][t].
//
// Unit (head hq, slice s) takes all M tokens of one query head against one key slice
// (verify_slices); units are numbered u = (j * nsl + s) * NKV + g for head j of KV group g, so
// with workgroups dealt round-robin over the 8 XCDs the units of one group read its K / V rows
// through one L2. The unit's cached K / V rows are requested before the wait for q. Per 16-key
// chunk and 16-token row tile a wave forms S^T = K Q^T with two 16x16x32 bf16 MFMAs (lane (r, c)
// then holds the scores of token r for keys 4c .. 4c+3), updates the rows' running max and sum
// (exp2 domain), and accumulates O^T = V^T P^T with 16x16x16 bf16 MFMAs, P split into three bf16
// terms p = hi + mid + lo (each product with a bf16 value exact in fp32, so the accumulation is
// fp32 p.v up to summation order). The waves that split one row tile's chunks merge through LDS.
// With one unit per head it writes bf16(o / sum) to vattn itself; otherwise every unit publishes
// each token's (max, sum, o[64]) as tagged fp32 words, then merges the tokens m = s, s + nsl, ...
// over the head's units in unit order and writes them. Each unit then sets its ready flag
// (VF_ATTN + hq * nsl + s). Timestamps (slot, 4 per call): q staged, keys done, partials
// published (or output written), flag set.
__device__ void attention_verify(const DecodeParams& p, int l, uint32_t qtag, uint32_t otag,
                                 unsigned char* ua, int& slot) {
  const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, c = lane >> 4;
  const int M = p.M, pos = p.pos, NH = p.NH, NKV = p.NKV, QPG = p.NH / p.NKV, G = grid_here();
  const int HALF = (NH + 2 * NKV) * 32;  // tagged pairs per token
  const int RT = (M + 15) >> 4;          // token row tiles (1 or 2)
  int nsl, kps;
  verify_slices(p, pos, NH, G, nsl, kps);
  const float sc = p.attn_scale * 1.4426950408889634f;
  uint16_t* const qs = reinterpret_cast<uint16_t*>(ua + VA_Q);
  uint16_t* const ks = reinterpret_cast<uint16_t*>(ua + VA_K);
  uint16_t* const vt = reinterpret_cast<uint16_t*>(ua + VA_VT);
  uint8_t* const amk = ua + VA_MASK;
  float* const wp = reinterpret_cast<float*>(ua + VA_WP);
  unsigned long long* const vpart = p.vpart;  // [NH][VNS][32][66] tagged fp32
  int WPR = 1;  // waves per row tile
  while (RT * WPR * 2 <= NWAVE) WPR *= 2;
  const int myrt = wave % RT, kp = wave / RT;  // this wave's row tile and chunk phase
  const int nunits = NH * nsl;
  if ((int)blockIdx.x >= nunits) {
    stamp(p, slot);
    stamp(p, slot);
    stamp(p, slot);
  }
  for (int unit = blockIdx.x; unit < nunits; unit += G) {
    const int g = unit % NKV, rest = unit / NKV, sl = rest % nsl, jh = rest / nsl;
    const int hq = g * QPG + jh;
    const bool last = sl == nsl - 1;  // also takes the new keys
    const int k0 = sl * kps, nc = max(0, min(pos, k0 + kps) - k0);  // cached keys of the unit
    const int nk = nc + (last ? M : 0);
    const size_t cbase = (size_t)(l * NKV + g) * p.S * 64;
    // cached keys [k0 + kb, k0 + kb + n) into rows 0 .. n-1 of ks and columns 0 .. n-1 of vt
    auto load_round = [&](int kb, int n) {
      const auto kr = buf_rsrc(p.kc + cbase + (size_t)(k0 + kb) * 64, (uint32_t)n * 128u);
      const auto vr = buf_rsrc(p.vc + cbase + (size_t)(k0 + kb) * 64, (uint32_t)n * 128u);
      uint4 kv[4], vv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // VRK * 8 = 2048 16-byte chunks each of K and V: 4 per thread
        const int ci = tid + NT * i;
        kv[i] = buf_ld128(kr, (uint32_t)ci * 16u);
        vv[i] = buf_ld128(vr, (uint32_t)ci * 16u);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ci = tid + NT * i, key = ci >> 3, d0 = (ci & 7) * 8;
        if (key >= n) continue;  // rows past the round: the new keys may be staged there
        *reinterpret_cast<uint4*>(ks + key * 64 + d0) = kv[i];
        const uint32_t w4[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vt[(d0 + 2 * e) * VT_LD + key] = (uint16_t)w4[e];
          vt[(d0 + 2 * e + 1) * VT_LD + key] = (uint16_t)(w4[e] >> 16);
        }
      }
    };
    // (the first round is stored before the q wait: holding it in registers across the wait, as
    // the decode kernel's by-group attention does, spills in this kernel)
    if (nc > 0) load_round(0, min(nc, VRK));  // cached keys: requested before the q wait
    // q of the head for every token (zero rows up to the tile edge); for the last slice the new
    // keys' K / V rows (after the round's cached keys, if they fit, else in a round of their own)
    // and the mask
    const int nb0 = (nc + M <= VRK) ? nc : 0;  // where the new keys go in ks / vt
    {
      const int nq = M * 32, nkv = last && nb0 == nc ? 64 * M : 0, total = nq + nkv;
      constexpr int B = 4;
      auto word = [&](int idx) {  // tagged pair of item idx: q pairs, then new k, then new v
        if (idx < nq) return p.qkv + (size_t)(idx >> 5) * HALF + hq * 32 + (idx & 31);
        const int i2 = idx - nq, which = i2 / (32 * M), r2 = i2 - which * 32 * M;
        return p.qkv + (size_t)(r2 >> 5) * HALF + (which ? NH + NKV + g : NH + g) * 32 + (r2 & 31);
      };
      for (int base = 0; base < total; base += B * NT) {
        unsigned long long v[B];
#pragma unroll
        for (int i = 0; i < B; ++i) {
          const int idx = base + tid + i * NT;
          v[i] = idx < total ? ld_coh_u64(word(idx)) : 0ull;
        }
        poll_tagged<B>(p, v, qtag, [&](int i) { return word(base + tid + i * NT); },
                       [&](int i) { return base + tid + i * NT < total; });
#pragma unroll
        for (int i = 0; i < B; ++i) {
          const int idx = base + tid + i * NT;
          if (idx < total) {
            const uint16_t lo = (uint16_t)v[i], hi = (uint16_t)(v[i] >> 16);
            if (idx < nq) {
              const int m = idx >> 5, dp = idx & 31;
              qs[m * 64 + dp] = lo;
              qs[m * 64 + dp + 32] = hi;
            } else {
              const int i2 = idx - nq, which = i2 / (32 * M), r2 = i2 - which * 32 * M;
              const int t = nb0 + (r2 >> 5), dp = r2 & 31;
              if (which == 0) {
                ks[t * 64 + dp] = lo;
                ks[t * 64 + dp + 32] = hi;
              } else {
                vt[dp * VT_LD + t] = lo;
                vt[(dp + 32) * VT_LD + t] = hi;
              }
            }
          }
        }
      }
      for (int i = tid; i < (RT * 16 - M) * 32; i += NT) reinterpret_cast<uint32_t*>(qs + M * 64)[i] = 0u;
      if (last)
        for (int i = tid; i < M * M; i += NT) amk[i] = p.amask[i];
    }
    lds_barrier();
    stamp(p, slot);
    // ---- S, online softmax and P.V, one round of keys at a time: ncr cached keys (rows 0 ..
    // ncr-1 of ks / vt), then, in the round that holds them, the M new keys (rows ncr .. ncr+M-1)
    float mrun = -INFINITY, lrun = 0.0f;
    fl_f32x4 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = fl_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const bool active = wave < RT * WPR;
    const uint16_t* qrow = qs + (myrt * 16 + r) * 64 + c * 8;
    const int mrow = min(myrt * 16 + r, M - 1);  // this lane's token (rows past M are padding)
    // value columns past the round's keys up to the chunk edge must be finite (p = 0 there)
    auto zero_tail = [&](int nr) {
      for (int i = tid; i < 64 * 16; i += NT) {
        const int col = nr + (i & 15);
        if (col < ((nr + 15) & ~15)) vt[(i >> 4) * VT_LD + col] = 0;
      }
    };
    int kb = 0, ncr = min(VRK, nc);
    bool new_in = last && nb0 == nc, new_done = !last || nb0 == nc;
    zero_tail(ncr + (new_in ? M : 0));
    lds_barrier();
    for (;;) {
      const int nr = ncr + (new_in ? M : 0);
      if (active && nr > 0) {
        const uint4 qa = *reinterpret_cast<const uint4*>(qrow);
        const uint4 qb = *reinterpret_cast<const uint4*>(qrow + 32);
        for (int ch = kp; ch * 16 < nr; ch += WPR) {
          const uint16_t* krow = ks + (ch * 16 + r) * 64 + c * 8;
          fl_f32x4 st = {0.0f, 0.0f, 0.0f, 0.0f};
          st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(fl_bf16x8, *reinterpret_cast<const uint4*>(krow)),
              __builtin_bit_cast(fl_bf16x8, qa), st, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(fl_bf16x8, *reinterpret_cast<const uint4*>(krow + 32)),
              __builtin_bit_cast(fl_bf16x8, qb), st, 0, 0, 0);
          // st[i]: score of token row r, round key ch * 16 + 4c + i
          float sv[4], mx = -INFINITY;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kl = ch * 16 + 4 * c + i;
            bool ok = kl < nr;
            if (kl >= ncr) ok = ok && amk[mrow * M + min(kl - ncr, M - 1)] != 0;  // a new key
            sv[i] = ok ? st[i] * sc : -INFINITY;
            mx = fmaxf(mx, sv[i]);
          }
          mx = xor32_max(xor16_max(mx));
          const float mn = fmaxf(mrun, mx);
          const float mu = (mn == -INFINITY) ? 0.0f : mn;
          const float corr = __builtin_amdgcn_exp2f(mrun - mu);
          float pv[4];
          float ps = 0.0f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pv[i] = __builtin_amdgcn_exp2f(sv[i] - mu);
            ps += pv[i];
          }
          ps = xor32_sum(xor16_sum(ps));
          lrun = lrun * corr + ps;
          mrun = mn;
          uint32_t ph[2], pm[2], pl[2];  // p = hi + mid + lo, three bf16 terms
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float a0 = pv[2 * e], a1 = pv[2 * e + 1];
            ph[e] = pack_bf16x2(a0, a1);
            const float r0 = a0 - bflo(ph[e]), r1 = a1 - bfhi(ph[e]);
            pm[e] = pack_bf16x2(r0, r1);
            pl[e] = pack_bf16x2(r0 - bflo(pm[e]), r1 - bfhi(pm[e]));
          }
          typedef short fl_s16x4 __attribute__((ext_vector_type(4)));
          const fl_s16x4 bh = __builtin_bit_cast(fl_s16x4, make_uint2(ph[0], ph[1]));
          const fl_s16x4 bm = __builtin_bit_cast(fl_s16x4, make_uint2(pm[0], pm[1]));
          const fl_s16x4 bl = __builtin_bit_cast(fl_s16x4, make_uint2(pl[0], pl[1]));
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            fl_f32x4 acc = o[dt];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] *= corr;
            const fl_s16x4 va = __builtin_bit_cast(
                fl_s16x4, *reinterpret_cast<const uint2*>(vt + (dt * 16 + r) * VT_LD + ch * 16 + 4 * c));
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, bm, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, bl, acc, 0, 0, 0);
            o[dt] = acc;
          }
        }
      }
      if (kb + VRK < nc) {  // the next round of cached keys
        lds_barrier();      // every wave is done with this one
        kb += VRK;
        ncr = min(VRK, nc - kb);
        load_round(kb, ncr);
        zero_tail(ncr);
        lds_barrier();
      } else if (!new_done) {  // the new keys in a round of their own (rows 0 .. M-1)
        lds_barrier();
        for (int i = tid; i < 64 * M; i += NT) {
          const int which = i / (32 * M), r2 = i - which * 32 * M, t = r2 >> 5, dp = r2 & 31;
          const unsigned long long w =
              wait_pair(p, p.qkv + (size_t)t * HALF + (which ? NH + NKV + g : NH + g) * 32 + dp, qtag);
          if (which == 0) {
            ks[t * 64 + dp] = (uint16_t)w;
            ks[t * 64 + dp + 32] = (uint16_t)(w >> 16);
          } else {
            vt[dp * VT_LD + t] = (uint16_t)w;
            vt[(dp + 32) * VT_LD + t] = (uint16_t)(w >> 16);
          }
        }
        ncr = 0;
        new_in = new_done = true;
        zero_tail(M);
        lds_barrier();
      } else {
        break;
      }
    }
    stamp(p, slot);
    // ---- the unit's (max, sum, o) per token: the WPR waves of each row tile merge through LDS
    // (o[dt][i] at lane (r, c): token row r, dim 16 dt + 4 c + i)
    lds_barrier();
    if (active) {
      float* w = wp + (wave * 16 + r) * 66;
      if (c == 0) {
        w[0] = mrun;
        w[1] = lrun;
      }
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) w[2 + dt * 16 + 4 * c + i] = o[dt][i];
    }
    lds_barrier();
    // thread (token m, word wd): the unit's value of that word, waves of the row tile in order
    auto unit_word = [&](int m, int wd) {
      const int rt = m >> 4, rr = m & 15;
      float mm = -INFINITY;
      for (int q = 0; q < WPR; ++q) mm = fmaxf(mm, wp[((rt + q * RT) * 16 + rr) * 66]);
      if (wd == 0) return mm;
      float val = 0.0f;
      for (int q = 0; q < WPR; ++q) {
        const float* w = wp + ((rt + q * RT) * 16 + rr) * 66;
        const float e = (w[0] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(w[0] - mm);
        val += w[wd] * e;
      }
      return val;
    };
    unsigned long long* const hp = vpart + (size_t)hq * VNS * FL_MAX_VERIFY * 66;
    uint32_t* const flag = p.vflag + VF_ATTN + hq * nsl + sl;
    if (nsl == 1) {  // the unit saw every key: its rows are the output
      for (int it = tid; it < M * 64; it += NT) {
        const int m = it >> 6, d = it & 63;
        st_coh_u16(p.vattn + (size_t)m * p.D + hq * 64 + d, f2bf(unit_word(m, 2 + d) / unit_word(m, 1)));
      }
      stamp(p, slot);
      set_flag(flag, otag);
    } else {
      // publish every token's (max, sum, o), then merge the tokens m = sl, sl + nsl, ... over the
      // head's nsl units: thread (token of pass q and wave, dim d), words of the units in order
      for (int it = tid; it < M * 66; it += NT) {
        const int m = it / 66, wd = it - m * 66;
        st_coh_u64(hp + ((size_t)sl * FL_MAX_VERIFY + m) * 66 + wd,
                   (unsigned long long)__float_as_uint(unit_word(m, wd)) | ((unsigned long long)otag << 32));
      }
      stamp(p, slot);
      const int ntok = (M - sl + nsl - 1) / nsl, npass = (ntok + NWAVE - 1) / NWAVE;  // <= 4
      const int d = lane;
      auto tok = [&](int q) { return sl + (q * NWAVE + wave) * nsl; };
      // words 0 .. VNS-1: o[d] of (pass i / nsl, unit i % nsl), npass * nsl <= VNS; VNS + q: (d < 2 nsl)
      // max / sum of unit d / 2 for pass q
      unsigned long long wv[VNS + 4];
      auto valid = [&](int i) {
        if (i < VNS) return i < npass * nsl && tok(i / nsl) < M;
        return i - VNS < npass && tok(i - VNS) < M && d < 2 * nsl;
      };
      auto addr = [&](int i) {
        return i < VNS ? hp + ((size_t)(i % nsl) * FL_MAX_VERIFY + tok(i / nsl)) * 66 + 2 + d
                       : hp + ((size_t)(d >> 1) * FL_MAX_VERIFY + tok(i - VNS)) * 66 + (d & 1);
      };
#pragma unroll
      for (int i = 0; i < VNS + 4; ++i) wv[i] = valid(i) ? ld_coh_u64(addr(i)) : 0ull;
      poll_tagged<VNS + 4>(p, wv, otag, addr, valid);
      float* const mlw = reinterpret_cast<float*>(ks);  // [4][NWAVE][VNS][2] max, sum
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (valid(VNS + q)) mlw[((q * NWAVE + wave) * VNS + (d >> 1)) * 2 + (d & 1)] = __uint_as_float((uint32_t)wv[VNS + q]);
      lds_barrier();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (q < npass && tok(q) < M) {
          const float* ml = mlw + (q * NWAVE + wave) * VNS * 2;
          float mm = -INFINITY;
          for (int u = 0; u < nsl; ++u) mm = fmaxf(mm, ml[2 * u]);
          float L = 0.0f, O = 0.0f;
#pragma unroll
          for (int i = 0; i < VNS; ++i) {
            if (i / nsl == q && i < npass * nsl) {
              const int u = i % nsl;
              const float e = (ml[2 * u] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ml[2 * u] - mm);
              L += ml[2 * u + 1] * e;
              O += __uint_as_float((uint32_t)wv[i]) * e;
            }
          }
          st_coh_u16(p.vattn + (size_t)tok(q) * p.D + hq * 64 + d, f2bf(O / L));
        }
      }
      set_flag(flag, otag);
    }
    lds_barrier();
  }
  stamp(p, slot);
}

// Which verify attention runs: by tokens (no merge across workgroups; each unit runs its tokens
// over every key of its head, two per pass) while w x keys is at most p.vtok_work (5120), with
// w = 1 for units of one or two tokens (a pair costs about one token) and w = tokens per unit
// above; else by key slices (matrix cores, merged over the slices). Measured on the 3B shape
// (40 heads, 256 workgroups, ctx 512-4096) the two meet at ctx ~5000 for M <= 12 (1 or 2 tokens
// per unit), ~1800 for M = 16 (3), ~1450 for M = 24 (4) and ~750 for M = 32 (6). Returns the
// number of ready flags its units set.
// The host picks the k_verify instantiation by this rule (each holds one of the two attentions:
// the slice attention alone is 35 KB of code, and without it the by-tokens layer loop fits the
// instruction cache far better).
__host__ __device__ inline bool verify_by_tokens(int NH, int M, int pos, int G, int vtok_work) {
  int tpu, ngrp;
  verify_units(NH, M, G, tpu, ngrp);
  const int w = tpu <= 2 ? 1 : tpu;
  return w * (pos > 1 ? pos : 1) <= vtok_work && NH * ngrp <= VF_ACT - VF_ATTN;
}
// ready flags the attention units of mode AM (1: by tokens, 2: by key slices) set
template <int AM>
__device__ __forceinline__ int verify_attn_flags(const DecodeParams& p) {
  const int G = grid_here();
  if constexpr (AM == 1) {
    int tpu, ngrp;
    verify_units(p.NH, p.M, G, tpu, ngrp);
    return p.NH * ngrp;
  } else {
    int nsl, kps;
    verify_slices(p, p.pos, p.NH, G, nsl, kps);
    return p.NH * nsl;
  }
}

template <int AM>  // attention by tokens (1) or by key slices (2), as verify_by_tokens picks
__global__ __launch_bounds__(NT, 1) void k_verify(DecodeParams pv) {
  (void)pv;  // read through params_here()
  const DecodeParams& p = params_here();
  extern __shared__ __align__(16) unsigned char vsm[];
  const int tid = threadIdx.x, wg = blockIdx.x, G = gridDim.x;
  const int D = p.D, F = p.F, NH = p.NH, NKV = p.NKV, M = p.M, pos = p.pos;
  const int NQKV = (NH + 2 * NKV) * 64, HALF = NQKV / 2;
  const int ld = D + 8;
  uint16_t* xs = reinterpret_cast<uint16_t*>(vsm);  // also the attention unit's region
  uint16_t* nws = reinterpret_cast<uint16_t*>(vsm + verify_xs_bytes(D));  // RMSNorm weights [D]
  float* part = reinterpret_cast<float*>(vsm + verify_xs_bytes(D) + verify_nw_bytes(D));
  uint16_t* hres = reinterpret_cast<uint16_t*>(part + VPART_TILES * NWAVE * 256);  // [FL_MAX_VERIFY][16]
  for (int i = tid; i < (ld >> 3); i += NT) reinterpret_cast<uint4*>(xs + VH * ld)[i] = make_uint4(0u, 0u, 0u, 0u);
  int slot = 0;  // optional timestamps, same slots as k_decode's
  stamp(p, slot);
  if (p.stall && wg == 0 && tid == 0) (void)wait_u32(p, p.stall, 1u);  // forced timeout (tests)

  auto token_at = [&](int m) {
    int t = p.tokens[m];
    if (t < 0 || t >= p.V) {
      if (tid == 0 && wg == 0)
        __hip_atomic_store(p.err, (int32_t)FL_E_ARG, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      t = 0;
    }
    return t;
  };
  auto rope_pos = [&](int m) {
    int r = pos + p.depth[m];
    if (r < 0 || r >= p.w.rope_len) {
      if (tid == 0 && wg == 0)
        __hip_atomic_store(p.err, (int32_t)FL_E_POS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      r = min(max(r, 0), p.w.rope_len - 1);
    }
    return r;
  };
  // this workgroup owns rows 16 wg .. 16 wg + 15 of h (its O tile and its down tile): their
  // values for every token stay in LDS, starting from bf16(embed[token] * emb_mult) (model.py:138)
  const bool owner = wg < D / 16;
  if (owner)
    for (int i = tid; i < M * 16; i += NT)
      hres[i] = (uint16_t)f2bf(rbf(bf2f(p.w.embed[(size_t)token_at(i >> 4) * D + wg * 16 + (i & 15)]) * p.emb_mult));

  for (int l = 0; l < params_here().NL; ++l) {
    const DecodeParams& p = params_here();
    const uint32_t e0 = p.epoch + 5u * (uint32_t)l;
    const uint32_t t_prev = tag_of(e0 - 1), t_qkv = tag_of(e0), t_attn = tag_of(e0 + 1),
                   t_h1 = tag_of(e0 + 2), t_act = tag_of(e0 + 3), t_h2 = tag_of(e0 + 4);
    uint32_t* const vf = p.vflag;
    // ---------------- P1: RMSNorm + QKV + RoPE + KV append ----------------
    const uint32_t* const qkv_q = p.w.wqkv_t + (size_t)l * NQKV * (D >> 3);  // tiled layout
    const uint32_t* const qkv_sz = p.w.wqkv_sz + (size_t)l * NQKV * (D >> 7);
    if (wg < NQKV / 16) {
      stage_norm_w(p.w.attn_norm + (size_t)l * D, D, nws);
      for (int h0 = 0; h0 < M; h0 += VH) {
        const int mh = min(VH, M - h0);
        TileW tw;
        tile_load(qkv_q, qkv_sz, wg * 16, 16, D, 0, D >> 7, tw);
        if (l == 0) {  // bf16(embed[token] * emb_mult)  (engine/model.py:138)
          if (h0 > 0) lds_barrier();  // every wave is done with the previous pass's rows
          for (int i = tid; i < mh * (D >> 1); i += NT) {
            const int m = i / (D >> 1), c = i - m * (D >> 1);
            const uint32_t e2 = reinterpret_cast<const uint32_t*>(p.w.embed + (size_t)token_at(h0 + m) * D)[c];
            reinterpret_cast<uint32_t*>(xs + m * ld)[c] =
                pack_bf16x2(rbf(bflo(e2) * p.emb_mult), rbf(bfhi(e2) * p.emb_mult));
          }
          lds_barrier();
          norm_rows(xs, ld, mh, D, nws, p.eps, part);
          lds_barrier();
        } else {
          if (h0 == 0) wait_flags(p, vf + VF_H2, D / 16, t_prev);
          else lds_barrier();
          stage_norm_rows(p.vh, h0, mh, D, xs, ld, nws, p.eps, part);
        }
        if (h0 == 0) stamp(p, slot);
        for (int t = wg; t < NQKV / 16; t += G) {
          const int n0 = t * 16;
          const TileW cur = tw;
          if (t + G < NQKV / 16) tile_load(qkv_q, qkv_sz, (t + G) * 16, 16, D, 0, D >> 7, tw);
          fl_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
          tile_mma(cur, D >> 7, xs, ld, mh, acc);
          tile_publish(part, acc);
          if (tid < 128) {  // (token, NEOX pair) of the tile
            const int ml = tid >> 3, pp = tid & 7, m = h0 + ml;
            if (ml < mh) {
              const float a = rbf(tile_sum(part, ml * 16 + 2 * pp)), b = rbf(tile_sum(part, ml * 16 + 2 * pp + 1));
              const int srow = n0 + 2 * pp;
              const int hh = srow >> 6, j = (srow & 63) >> 1;
              float oa = a, ob = b;
              if (hh < NH + NKV) {  // RoPE at pos + depth[m] (engine/model.py:257-269)
                const uint32_t cs = reinterpret_cast<const uint32_t*>(p.w.rope)[rope_pos(m) * 32 + j];
                const float cc = bflo(cs), sn = bfhi(cs);
                oa = rbf(a * cc - b * sn);
                ob = rbf(b * cc + a * sn);
              }
              st_coh_u64(p.qkv + (size_t)m * HALF + hh * 32 + j,
                         (unsigned long long)pack_bf16x2(oa, ob) | ((unsigned long long)t_qkv << 32));
              if (hh >= NH) {  // KV append at slot pos + m
                const int g = (hh < NH + NKV) ? hh - NH : hh - NH - NKV;
                uint16_t* dst = ((hh < NH + NKV) ? p.kc : p.vc) + ((size_t)(l * NKV + g) * p.S + pos + m) * 64;
                dst[j] = (uint16_t)f2bf(oa);
                dst[j + 32] = (uint16_t)f2bf(ob);
              }
            }
          }
          lds_barrier();
        }
      }
    } else {
      stamp(p, slot);
    }
    stamp(p, slot);
    // ---------------- P2: attention ----------------
    if constexpr (AM == 1) attention_verify_tokens(p, l, t_qkv, t_attn, vsm, slot);
    else attention_verify(p, l, t_qkv, t_attn, vsm, slot);
    // the attention unit used the staged-rows region: the zero row again
    for (int i = tid; i < (ld >> 3); i += NT) reinterpret_cast<uint4*>(xs + VH * ld)[i] = make_uint4(0u, 0u, 0u, 0u);
    // ---------------- P3: O projection + residual ----------------
    if (owner) {
      const uint32_t* const o_q = p.w.wo_t + (size_t)l * D * (D >> 3);  // tiled layout
      const uint32_t* const o_sz = p.w.wo_sz + (size_t)l * D * (D >> 7);
      for (int h0 = 0; h0 < M; h0 += VH) {
        const int mh = min(VH, M - h0);
        TileW tw;
        tile_load(o_q, o_sz, wg * 16, 16, D, 0, D >> 7, tw);  // before the wait, as every phase's tiles
        if (h0 == 0) {
          wait_flags(p, vf + VF_ATTN, verify_attn_flags<AM>(p), t_attn);
        } else {
          lds_barrier();
        }
        stage_bf16(p.vattn, D, h0, mh, 0, D, xs, ld);
        lds_barrier();
        if (h0 == 0) stamp(p, slot);
        fl_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        tile_mma(tw, D >> 7, xs, ld, mh, acc);
        tile_publish(part, acc);
        if (tid < 256) {
          const int ml = tid >> 4, n = tid & 15, m = h0 + ml;
          if (ml < mh) {  // h1 = bf16(h + bf16(bf16(o) * rm))  (engine/model.py:162)
            const float o = rbf(rbf(tile_sum(part, tid)) * p.resid_mult);
            const uint32_t h1 = f2bf(bf2f(hres[m * 16 + n]) + o);
            hres[m * 16 + n] = (uint16_t)h1;
            st_coh_u16(p.vh + (size_t)m * D + wg * 16 + n, h1);
          }
        }
        lds_barrier();
      }
      set_flag(vf + VF_H1 + wg, t_h1);
    }
    // ---------------- P4: RMSNorm + gate/up + SwiGLU ----------------
    if (!owner) stamp(p, slot);
    stamp(p, slot);
    if (wg < (2 * F) / 16) {
      const uint32_t* const gu_q = p.w.wgu_t + (size_t)l * 2 * F * (D >> 3);  // tiled layout
      const uint32_t* const gu_sz = p.w.wgu_sz + (size_t)l * 2 * F * (D >> 7);
      // this workgroup's tiles wg, wg+G, ... in rounds of up to 4: the round's MFMAs run back to
      // back into 4 accumulators, one publish and one epilogue per round. The first round's
      // weights are requested before the input wait, each later round's during the one before.
      const int nt = ((2 * F) / 16 - wg + G - 1) / G;
      stage_norm_w(p.w.ffn_norm + (size_t)l * D, D, nws);
      for (int h0 = 0; h0 < M; h0 += VH) {
        const int mh = min(VH, M - h0);
        const bool last = h0 + VH >= M;
        // the four tiles' weights requested before the input wait (they arrive during it; the
        // rows queue behind them)
        TileW tw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)  // tiles past nt: an empty range, no memory access
          tile_load(gu_q, gu_sz, (wg + i * G) * 16, i < nt ? 16 : 0, D, 0, D >> 7, tw[i]);
        if (h0 == 0) wait_flags(p, vf + VF_H1, D / 16, t_h1);
        else lds_barrier();
        stage_norm_rows(p.vh, h0, mh, D, xs, ld, nws, p.eps, part);
        if (h0 == 0) stamp(p, slot);
        for (int b4 = 0; b4 < nt; b4 += 4) {
          fl_f32x4 acc[4] = {};
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (b4 + i < nt) tile_mma(tw[i], D >> 7, xs, ld, mh, acc[i]);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (b4 + i + 4 < nt) tile_load(gu_q, gu_sz, (wg + (b4 + i + 4) * G) * 16, 16, D, 0, D >> 7, tw[i]);
          tile_publish4(part, acc);
          for (int it = tid; it < 4 * 128; it += NT) {
            const int i = it >> 7, ml = (it >> 3) & 15, pp = it & 7;
            if (b4 + i < nt && ml < mh) {  // act = bf16(bf16(silu(g)) * u)  (engine/model.py:227-228)
              const float* pt = part + i * NWAVE * 256;
              const float gg = rbf(tile_sum(pt, ml * 16 + 2 * pp)), uu = rbf(tile_sum(pt, ml * 16 + 2 * pp + 1));
              const int n0 = (wg + (b4 + i) * G) * 16;
              st_coh_u16(p.vact + (size_t)(h0 + ml) * F + (n0 >> 1) + pp, f2bf(rbf(silu_f(gg)) * uu));
            }
          }
          if (last) {  // the round's tiles are written for every token: their ready flags
            release_rows();
            if (tid < 4 && b4 + tid < nt) st_coh_u32(vf + VF_ACT + wg + (b4 + tid) * G, t_act << 16);
          } else {
            lds_barrier();
          }
        }
      }
    }
    if (wg >= (2 * F) / 16) stamp(p, slot);
    stamp(p, slot);
    // ---------------- P5: down projection + residual, K split over workgroups ----------------
    // The 8192-long K of each 16-row tile is cut into parts of 8 groups (1024 inputs; fewer when
    // D < 1024, as a part is staged into one xs row), one group per wave. Workgroup w takes part
    // k = w % KP of the tiles w / KP, w / KP + G / KP, ...: it stages only its part's inputs (those
    // of the gate/up tiles behind them, by their ready flags), runs one group per wave for each of
    // its tiles (weights requested once its inputs are in), and publishes each tile's part sum
    // (fp32, tagged) to p.part. The tile's owner (workgroup t) sums the parts in order and adds
    // the residual.
    int p5slot = slot;
    slot += 2;
    {
      const uint32_t* const d_q = p.w.wd_t + (size_t)l * D * (F >> 3);  // tiled layout
      const uint32_t* const d_sz = p.w.wd_sz + (size_t)l * D * (F >> 7);
      const int ntile = D / 16, ng = F >> 7, GPP = min(NWAVE, D >> 7), KP = (ng + GPP - 1) / GPP, GK = G / KP;
      const int k = wg % KP, kg0 = k * GPP, kgn = min(GPP, ng - kg0);
      const int nmine = (wg < GK * KP) ? max(0, (ntile - wg / KP + GK - 1) / GK) : 0;
      unsigned long long* const dpart = p.part;  // [tile][part][FL_MAX_VERIFY][16]
      constexpr int R = VPART_TILES, TMAX = 2 * R;  // tiles per round; tiles requested together
      for (int h0 = 0; h0 < M; h0 += VH) {
        const int mh = min(VH, M - h0);
        TileW1 tw[TMAX] = {};
        if (nmine > 0) {
          // the tiles' weights before the input wait, then each lane's own activation fragment
          // (a wave's MFMA reads only its K group) into the LDS place tile_mma1 reads it from:
          // every lane reads back only what it wrote, so no barrier
#pragma unroll
          for (int i = 0; i < TMAX; ++i)
            if (i < nmine) tile_load1(d_q, d_sz, (wg / KP + i * GK) * 16, F, kg0, kgn, tw[i]);
          if (h0 == 0) wait_flags(p, vf + VF_ACT + 16 * kg0, 16 * kgn, t_act);  // gate/up tiles of this part
          else lds_barrier();  // every wave is done with the previous pass's fragments
          stage_frag(p.vact, F, h0, mh, kg0 * 128, kgn, xs, ld);
          if (h0 == 0) stamp(p, p5slot);
        }
        for (int j0 = 0; j0 < nmine; j0 += R) {
          if (j0 >= TMAX) {  // more tiles than prefetched (few workgroups): one round at a time
#pragma unroll
            for (int i = 0; i < R; ++i)
              if (j0 + i < nmine) tile_load1(d_q, d_sz, (wg / KP + (j0 + i) * GK) * 16, F, kg0, kgn, tw[i]);
          }
          fl_f32x4 acc[R] = {};
#pragma unroll
          for (int i = 0; i < R; ++i)
            if (j0 + i < nmine) {
              const TileW1& w = j0 >= TMAX ? tw[i] : (j0 == 0 ? tw[i] : tw[R + i]);
              tile_mma1(w, kgn, xs, ld, mh, acc[i]);
            }
          tile_publish4(part, acc);
          for (int it = tid; it < R * 256; it += NT) {
            const int i = it >> 8, ml = (it >> 4) & 15, n = it & 15;
            if (j0 + i < nmine && ml < mh) {
              const int t = wg / KP + (j0 + i) * GK;
              const float v = tile_sum(part + i * NWAVE * 256, ml * 16 + n);
              st_coh_u64(dpart + (((size_t)t * KP + k) * FL_MAX_VERIFY + h0 + ml) * 16 + n,
                         (unsigned long long)__float_as_uint(v) | ((unsigned long long)t_h2 << 32));
            }
          }
          lds_barrier();
        }
      }
      if (nmine == 0) stamp(p, p5slot);
      // owner of tile wg: thread (m, n) sums its row's KP parts in order, h2 = h1 + bf16(bf16(d) * rm)
      if (owner) {
        if (tid < 16 * M) {
          const int m = tid >> 4, n = tid & 15;
          auto ok = [t_h2](unsigned long long v) { return (uint32_t)(v >> 32) == t_h2; };
          const unsigned long long* const a0 = dpart + ((size_t)wg * KP * FL_MAX_VERIFY + m) * 16 + n;
          constexpr size_t KS = (size_t)FL_MAX_VERIFY * 16;  // one part's stride
          float sum = 0.0f;
          bool in = false;
          if (KP <= 8 && M <= VH) {
            // one token pass: all parts requested at once; if one is not in yet, the parts are
            // read again below one at a time, each waited for (with several passes the parts
            // arrive spread out and the batch seldom finds them all: measured slower there)
            unsigned long long v8[8];
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) v8[kk] = kk < KP ? ld_coh_u64(a0 + kk * KS) : 0ull;
            in = true;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) in = in && (kk >= KP || ok(v8[kk]));
            if (__builtin_expect(in, 1)) {
#pragma unroll
              for (int kk = 0; kk < 8; ++kk)
                if (kk < KP) sum += __uint_as_float((uint32_t)v8[kk]);
            }
          }
          if (!in) {
            for (int kk = 0; kk < KP; ++kk) {
              const unsigned long long* a = a0 + kk * KS;
              unsigned long long v = ld_coh_u64(a);
              if (!ok(v)) v = spin_until(p, v, ok, [a]() { return ld_coh_u64(a); });
              sum += __uint_as_float((uint32_t)v);
            }
          }
          const float o = rbf(rbf(sum) * p.resid_mult);  // engine/model.py:163
          const uint32_t h2 = f2bf(bf2f(hres[m * 16 + n]) + o);
          hres[m * 16 + n] = (uint16_t)h2;
          st_coh_u16(p.vh + (size_t)m * D + wg * 16 + n, h2);
        }
        set_flag(vf + VF_H2 + wg, t_h2);
      }
    }
    stamp(p, p5slot);
  }

  // ---------------- final norm + tied bf16 LM head + per-token argmax ----------------
  const int ntile = (p.V + 15) / 16;
  const uint32_t t_fin = tag_of(p.epoch + 5u * (uint32_t)p.NL - 1u);
  for (int h0 = 0; h0 < M; h0 += VH) {
    const int mh = min(VH, M - h0);
    unsigned long long best = 0ull;
    if (wg < ntile || (p.feat && wg == 0)) {
      const int lane = tid & 63, wave = tid >> 6, r = lane & 15, c = lane >> 4;
      const int ksteps = D >> 5;
      const uint16_t* xrow = xs + (r < mh ? r : VH) * ld + c * 8;
      constexpr int SPW = 16;  // k-steps per wave (D <= 4096)
      // double-buffered: the next tile's embedding rows are requested before this tile's MFMAs; a
      // tile past the vocabulary requests nothing (empty range), so the loads stay branch-free
      auto load_tile = [&](int t, uint4 (&bw)[SPW]) {
        const int rows = max(0, min(16, p.V - t * 16));
        const auto er = buf_rsrc(p.w.embed + (size_t)t * 16 * D, (uint32_t)rows * (uint32_t)D * 2u);
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
          const int st = wave + NWAVE * i;
          bw[i] = buf_ld128(er, st < ksteps ? (uint32_t)(r * D + st * 32 + c * 8) * 2u : 0xFFFFFFF0u);
        }
      };
      auto do_tile = [&](int t, const uint4 (&bw)[SPW]) {
        const int n0 = t * 16, rows = min(16, p.V - n0);
        fl_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
          const int st = wave + NWAVE * i;
          if (st < ksteps) {
            const uint4 xa = *reinterpret_cast<const uint4*>(xrow + st * 32);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(fl_bf16x8, xa),
                                                          __builtin_bit_cast(fl_bf16x8, bw[i]), acc, 0, 0, 0);
          }
        }
        tile_publish(part, acc);
        if (tid < 256) {
          const int ml = tid >> 4, n = tid & 15;
          if (ml < mh && n < rows) {
            // logits = bf16(bf16(x . E^T) / logits_scaling)  (engine/model.py:144)
            const float lg = rbf(rbf(tile_sum(part, tid)) / p.logits_scaling);
            if (p.logits) p.logits[(size_t)(h0 + ml) * p.V + n0 + n] = lg;
            best = u64max(best, amax_key(lg, (uint32_t)(n0 + n)));
          }
        }
        lds_barrier();
      };
      uint4 bwa[SPW], bwb[SPW];
      load_tile(wg, bwa);  // the first tile's rows are requested before the input wait
      if (h0 == 0) {
        stage_norm_w(p.w.final_norm, D, nws);
        wait_flags(p, p.vflag + VF_H2, D / 16, t_fin);
      } else {
        lds_barrier();
      }
      stage_norm_rows(p.vh, h0, mh, D, xs, ld, nws, p.eps, part);
      if (h0 == 0) stamp(p, slot);
      if (p.feat && wg == 0)
        for (int i = tid; i < mh * D; i += NT) p.feat[(size_t)h0 * D + i] = xs[(i / D) * ld + (i % D)];
      for (int t = wg; t < ntile; t += 2 * G) {
        load_tile(t + G, bwb);
        do_tile(t, bwa);
        if (t + G >= ntile) break;
        load_tile(t + 2 * G, bwa);
        do_tile(t + G, bwb);
      }
    } else if (h0 == 0) {
      stamp(p, slot);
    }
    // per-token argmax: the 16 threads of a token row are lanes 16k..16k+15 of one wave
    if (tid < 256) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) best = u64max(best, (unsigned long long)__shfl_xor(best, o, 64));
      const int ml = tid >> 4;
      if ((tid & 15) == 0 && ml < mh && best != 0ull)
        __hip_atomic_fetch_max(p.amax + h0 + ml, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  stamp(p, slot);
  wait_mem();
  lds_barrier();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(p.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (uint32_t)(G - 1)) {
      for (int m = 0; m < M; ++m) {
        p.tokens_out[m] = (int32_t)amax_index(ld_coh_u64(p.amax + m));
        __hip_atomic_store(p.amax + m, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// KV cache compaction after a tree verify (the reference moves the accepted path's rows one
// index copy at a time, spec_tree.py:124-127). One workgroup per (layer, KV group): thread t of
// the first 16 n moves 16 bytes of K (t / 8 even) or V of row t / 16, and every row is read
// before any is written, so a destination that is also a later move's source is read first.
struct KvMove {
  int32_t src[FL_MAX_VERIFY], dst[FL_MAX_VERIFY];
  int32_t n;
};
// one workgroup per (layer, KV group); 16 threads per moved row (K and V, 8 x 16 bytes each)
constexpr int KV_MOVE_THREADS = 16 * FL_MAX_VERIFY;
__global__ __launch_bounds__(KV_MOVE_THREADS) void k_kv_move(uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                             int S, KvMove mv) {
  const int t = threadIdx.x;
  const size_t base = (size_t)blockIdx.x * S * 64;  // (layer, group) span: S rows of 64 bf16
  const int i = t >> 4, half = (t >> 3) & 1, part = t & 7;
  uint16_t* c = half ? vc : kc;
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  const bool on = i < mv.n;
  if (on) v = reinterpret_cast<const uint4*>(c + base + (size_t)mv.src[i] * 64)[part];
  __syncthreads();
  if (on) reinterpret_cast<uint4*>(c + base + (size_t)mv.dst[i] * 64)[part] = v;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// A GEMV phase's rows per workgroup fit its chunk budget: cap chunks per thread, dealt with
// mode GM_STRIDE (stride NT), GM_COLUMN (stride cs_stride(k): NT / (k / 32) rows of chunks per
// round), GM_ROWS (2^rs_lg lanes per row: ceil((k / 32) / lanes) chunks each) or GM_PAIRS
// (2^rp_lg lanes per row pair: twice that).
int phase_fits(int n, int k, int G, int cap, int mode) {
  int R = (n + G - 1) / G;
  R += (R & 1);
  const int cpr = k >> 5;
  if (R > ROWS_MAX || cpr > NT) return 0;
  // by rows / row pairs: at least 4 lanes per row, so each 4-lane block of the matrix-core
  // dequantisation stays on one row
  if (mode == GM_ROWS) {
    int lg = 5;  // rs_lg
    while (lg > 0 && ((R << lg) > NT || (1 << (lg - 1)) >= cpr)) --lg;
    return lg >= 2 && R <= NT && (cpr + (1 << lg) - 1) >> lg <= cap;
  }
  if (mode == GM_PAIRS) {
    const int lg = rp_lg(R, cpr);
    return lg >= 2 && R <= 2 * NT && 2 * ((cpr + (1 << lg) - 1) >> lg) <= cap;
  }
  return mode == GM_COLUMN ? R <= (NT / cpr) * cap : (long)R * cpr <= (long)cap * NT;
}

}  // namespace

struct fl_state {
  fl_model_desc d;
  int max_seq;
  int grid;   // decode workgroups (1 per CU)
  int vgrid;  // verify workgroups (1 per CU)
  uint16_t *kc, *vc;
  uint32_t *h, *attn, *act;
  unsigned long long* qkv;
  unsigned long long* part;
  uint16_t* vrows;              // verify exchange rows: h [FL_MAX_VERIFY][D], attn [..][D], act [..][F]
  unsigned long long* vpart;    // verify attention slice partials [NH][VNS][FL_MAX_VERIFY][66]
  uint32_t* vflag;              // verify ready flags
  uint32_t* shist;              // fused sampling exchange: per-workgroup histograms
  unsigned long long* sword;    // ... bin totals, maxima, partial sums
  int att_spw, gq_min, gq_kps;
  int defer_min;  // key slices from which the per-head attention leaves its merge to the O phase
  int vkps, vtok_work;
  int coop;       // launch with hipLaunchCooperativeKernel (else a plain launch, the default)
  // the k_decode instantiations of the chunk budget that fits the model, by attention: per-head
  // units (0), with the slice merge deferred to the O phase (1), by KV group (2; small budget only,
  // else null)
  const void* kdec[3];
  int verify_ok;  // k_verify's dynamic LDS fits and a grid of it is co-resident
  unsigned long long* amax;
  uint32_t* done;
  int32_t* err;
  uint32_t epoch;
  unsigned long long* prof;
  int prof_slots;
  unsigned long long spin_ticks;  // wait bound passed to every launch
  uint32_t* stall;                // zero word, never written: forced-timeout wait (tests)
  int force_timeout;
  void* blocks[16];
  int nblocks;
  void* uc[12];  // pooled uncached exchange buffers
  size_t uc_bytes[12];
  int nuc;
  // Tags are 16 bits (1..65535) and advance 5 per layer per launch, so a word left over from an
  // older launch could carry the tag a reader is waiting for once the tags have gone round. The
  // exchange buffers are zeroed (tag 0: never valid) every clear_period launches, fewer than
  // take the tags round.
  uint32_t clear_period, since_clear;
};

namespace {
__global__ __launch_bounds__(256) void k_zero(uint4* __restrict__ p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}
// zero every exchange buffer (a kernel, not hipMemsetAsync, so a captured stream stays valid)
int clear_exchange(fl_state* st, hipStream_t s) {
  for (int i = 0; i < st->nuc; ++i) {
    const size_t n16 = st->uc_bytes[i] / 16;
    hipLaunchKernelGGL(k_zero, dim3((unsigned)std::min<size_t>((n16 + 255) / 256, 4096)), dim3(256), 0, s,
                       reinterpret_cast<uint4*>(st->uc[i]), n16);
  }
  st->since_clear = 0;
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}
// after each decode / verify launch: 5 phases per layer. The epoch is kept reduced mod 65535 (the
// tag period), so the kernel's epoch + 5 * layer + phase never wraps the 32-bit range and every
// tag in a clear window stays distinct.
void advance_epoch(fl_state* st) {
  st->epoch = (st->epoch + 5u * (uint32_t)st->d.n_layer) % 65535u;
}
// before each decode / verify launch
int maybe_clear(fl_state* st, hipStream_t s) {
  return ++st->since_clear >= st->clear_period ? clear_exchange(st, s) : FL_OK;
}
template <typename T>
int dev_alloc(fl_state* st, T** p, size_t count) {
  void* v = nullptr;
  if (st->nblocks >= (int)(sizeof(st->blocks) / sizeof(st->blocks[0]))) return FL_E_ARG;
  if (hipMalloc(&v, count * sizeof(T) + 256) != hipSuccess) return FL_E_HIP;
  if (hipMemset(v, 0, count * sizeof(T) + 256) != hipSuccess) return FL_E_HIP;
  st->blocks[st->nblocks++] = v;
  *p = reinterpret_cast<T*>(v);
  return FL_OK;
}

// The tagged exchange buffers (activations handed between workgroups inside a launch) live in
// uncached device memory (hipDeviceMallocUncached). On gfx950 its lines are still held in the
// L2s, coherently (the exchange reads count as L2 hits, not as uncached requests or HBM reads);
// what it buys is that the device-coherent (sc1) stores and loads of the hand-offs need no L2
// write-back or invalidate, and it measured about 2% faster end to end than ordinary memory. Uncached memory is never freed
// once a kernel has read it (memory allocated after such a free has been seen to hold wrong
// values), so a destroyed state returns its blocks to this per-process pool, and later states on
// the same device reuse them, cleared (a stale tag must never match a new phase).
struct UcBlock {
  void* p;
  size_t bytes;
  int dev;
  bool used;
};
std::mutex g_uc_mu;
std::vector<UcBlock> g_uc;

template <typename T>
int uc_alloc(fl_state* st, T** p, size_t count) {
  const size_t bytes = count * sizeof(T) + 256;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FL_E_HIP;
  if (st->nuc >= (int)(sizeof(st->uc) / sizeof(st->uc[0]))) return FL_E_ARG;
  void* v = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_uc_mu);
    int best = -1;
    for (int i = 0; i < (int)g_uc.size(); ++i)
      if (!g_uc[i].used && g_uc[i].dev == dev && g_uc[i].bytes >= bytes &&
          (best < 0 || g_uc[i].bytes < g_uc[best].bytes))
        best = i;
    if (best >= 0) {
      g_uc[best].used = true;
      v = g_uc[best].p;
    } else {
      if (hipExtMallocWithFlags(&v, bytes, hipDeviceMallocUncached) != hipSuccess) return FL_E_HIP;
      g_uc.push_back(UcBlock{v, bytes, dev, true});
    }
  }
  if (hipMemset(v, 0, bytes) != hipSuccess) return FL_E_HIP;
  st->uc_bytes[st->nuc] = bytes;
  st->uc[st->nuc++] = v;
  *p = reinterpret_cast<T*>(v);
  return FL_OK;
}

void uc_release(void* v) {
  std::lock_guard<std::mutex> lk(g_uc_mu);
  for (auto& b : g_uc)
    if (b.p == v) b.used = false;
}
}  // namespace

namespace {
bool weights_ok(const fl_weights* w) {
  return w && w->wqkv_q && w->wqkv_sz && w->wo_q && w->wo_sz && w->wgu_q && w->wgu_sz && w->wd_q &&
         w->wd_sz && w->attn_norm && w->ffn_norm && w->final_norm && w->embed && w->rope &&
         w->rope_len > 0;
}

DecodeParams base_params(const fl_weights* w, fl_state* st, int pos) {
  DecodeParams p;
  memset(&p, 0, sizeof(p));
  p.w = *w;
  p.kc = st->kc;
  p.vc = st->vc;
  p.h = st->h;
  p.qkv = st->qkv;
  p.attn = st->attn;
  p.act = st->act;
  p.part = st->part;
  p.vh = st->vrows;
  p.vattn = st->vrows + (size_t)FL_MAX_VERIFY * st->d.dim;
  p.vact = st->vrows + (size_t)2 * FL_MAX_VERIFY * st->d.dim;
  p.vflag = st->vflag;
  p.vpart = st->vpart;
  p.shist = st->shist;
  p.sword = st->sword;
  p.att_spw = st->att_spw;
  p.gq_min = st->gq_min;
  p.gq_kps = st->gq_kps;
  p.vkps = st->vkps;
  p.vtok_work = st->vtok_work;
  p.amax = st->amax;
  p.done = st->done;
  p.err = st->err;
  p.D = st->d.dim;
  p.NH = st->d.n_head;
  p.NKV = st->d.n_kv_head;
  p.F = st->d.inter;
  p.V = st->d.vocab;
  p.NL = st->d.n_layer;
  p.S = st->max_seq;
  p.pos = pos;
  p.eps = st->d.norm_eps;
  p.emb_mult = st->d.emb_mult;
  p.attn_scale = st->d.attn_scale;
  p.resid_mult = st->d.resid_mult;
  p.logits_scaling = st->d.logits_scaling;
  p.epoch = st->epoch;
  p.spin_ticks = st->spin_ticks;
  p.stall = st->force_timeout ? st->stall : nullptr;
  p.M = 1;
  return p;
}
}  // namespace

namespace {
struct SampleArgs {
  float tdiv;  // 0: greedy
  int top_k;
  uint64_t seed, offset;
};
int decode_launch(const fl_weights* w, fl_state* st, const int32_t* token_in, uint16_t* h_io,
                  int32_t pos, int32_t* token_out, float* logits, uint16_t* feat, void* stream,
                  SampleArgs sa = SampleArgs{0.0f, 0, 0, 0}) {
  if (pos < 0 || pos >= st->max_seq || pos >= w->rope_len) return FL_E_POS;
  if (maybe_clear(st, as_stream(stream)) != FL_OK) return FL_E_LAUNCH;
  DecodeParams p = base_params(w, st, pos);
  p.samp_tdiv = sa.tdiv;
  p.samp_topk = sa.top_k;
  p.seed_lo = (uint32_t)sa.seed;
  p.seed_hi = (uint32_t)(sa.seed >> 32);
  p.off_lo = (uint32_t)sa.offset;
  p.off_hi = (uint32_t)(sa.offset >> 32);
  p.token_in = token_in;
  p.h_io = h_io;
  p.token_out = token_out;
  p.logits = logits;
  p.feat = feat;
  p.prof = st->prof;
  p.prof_slots = st->prof_slots;
  void* args[] = {&p};
  const void* kd = st->kdec[0];
  if (st->kdec[2] && gqa_applies(pos, st->gq_min, st->d.n_head, st->d.n_kv_head, st->grid)) {
    kd = st->kdec[2];
  } else {
    int nsl, sps;
    attn_slices(pos, st->d.n_head, st->grid, st->att_spw, nsl, sps);
    if (nsl >= st->defer_min) kd = st->kdec[1];
  }
  const hipError_t e =
      st->coop ? hipLaunchCooperativeKernel(kd, dim3(st->grid), dim3(NT), args, 0, as_stream(stream))
               : hipLaunchKernel(kd, dim3(st->grid), dim3(NT), args, 0, as_stream(stream));
  if (e != hipSuccess) return FL_E_LAUNCH;
  advance_epoch(st);
  return FL_OK;
}
}  // namespace

extern "C" {

int fl_device_info(int32_t* num_cu, int32_t* decode_grid) {
  int dev = 0, cu = 0, occ = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FL_E_HIP;
  if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return FL_E_HIP;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(k_decode<ChunksLarge, 0>),
                                                   NT, 0) != hipSuccess)
    return FL_E_HIP;
  if (num_cu) *num_cu = cu;
  if (decode_grid) *decode_grid = cu * (occ >= 1 ? 1 : 0);
  return FL_OK;
}

int fl_state_create(const fl_model_desc* d, int32_t max_seq, uint16_t* k_cache, uint16_t* v_cache,
                    fl_state** out) {
  if (!d || !out || !k_cache || !v_cache || max_seq <= 0) return FL_E_ARG;
  *out = nullptr;
  if (d->n_layer <= 0 || d->dim <= 0 || d->n_head <= 0 || d->n_kv_head <= 0 || d->inter <= 0 ||
      d->vocab <= 0)
    return FL_E_ARG;
  if (d->dim % FL_GROUP || d->inter % FL_GROUP || d->dim > XS_MAX || d->inter > XS_MAX ||
      d->dim > 64 * 8 * LM_MAXC || d->dim != d->n_head * FL_HEAD_DIM || d->n_head % d->n_kv_head)
    return FL_E_ARG;
  int dev = 0, cu = 0, occ = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FL_E_HIP;
  if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return FL_E_HIP;
  const int G = cu;
  const int D = d->dim, F = d->inter, NQKV = (d->n_head + 2 * d->n_kv_head) * FL_HEAD_DIM;
  auto fits = [&](auto c) {
    using C = decltype(c);
    return phase_fits(NQKV, D, G, C::QKV, C::ROWS ? GM_ROWS : GM_COLUMN) &&
           phase_fits(D, D, G, C::O, GM_COLUMN) &&
           phase_fits(2 * F, D, G, C::GU, C::ROWS ? GM_PAIRS : GM_STRIDE) &&
           phase_fits(D, F, G, C::D, GM_COLUMN);
  };
  // FLINT_AMD_DECODE_BUDGET=large selects the large-budget instantiation for any model (tests)
  const char* budget = getenv("FLINT_AMD_DECODE_BUDGET");
  const bool small = fits(ChunksSmall{}) && !(budget && strcmp(budget, "large") == 0);
  if (!small && !fits(ChunksLarge{})) return FL_E_ARG;
  const void* kdec[3] = {
      small ? reinterpret_cast<const void*>(k_decode<ChunksSmall, 0>) : reinterpret_cast<const void*>(k_decode<ChunksLarge, 0>),
      small ? reinterpret_cast<const void*>(k_decode<ChunksSmall, 1>) : reinterpret_cast<const void*>(k_decode<ChunksLarge, 1>),
      small ? reinterpret_cast<const void*>(k_decode<ChunksSmall, 2>) : nullptr};
  for (const void* k : kdec) {
    if (!k) continue;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, NT, 0) != hipSuccess) return FL_E_HIP;
    if (occ < 1 || cu < 1) return FL_E_LAUNCH;
  }
  fl_state* st = (fl_state*)calloc(1, sizeof(fl_state));
  if (!st) return FL_E_HIP;
  st->d = *d;
  st->max_seq = max_seq;
  st->grid = G;
  for (int i = 0; i < 3; ++i) st->kdec[i] = kdec[i];
  st->vgrid = cu;
  st->kc = k_cache;
  st->vc = v_cache;
  st->epoch = 1;
  {
    // epochs advance 5 * NL per launch; a tag repeats after 65535 epochs. Within a window of
    // P launches, 5 * NL * (P + 1) < 65535 keeps every (launch, layer, phase) tag distinct.
    long per = 5L * d->n_layer, P = 65535L / per - 2;
    if (const char* e = getenv("FL_CLEAR_PERIOD")) P = std::min(P, std::max(1L, atol(e)));  // tests
    st->clear_period = (uint32_t)std::max(1L, P);
    st->since_clear = 0;
  }
  st->att_spw = 7;  // one key slice up to 448 cached keys (tok/s at ctx 320 / 384 / 448: one slice
                    // 1136 / 1124 / 1112, five 1121 / 1119 / 1120)
  st->defer_min = DEFER_MERGE_SLICES;
  // the attention by KV group from 5120 cached keys: measured on one box against the per-head
  // units, +25 / +16 us per step at ctx 3072 / 4096, -13 / -20 / -17 us at 6144 / 8192 / 12288
  st->gq_min = 5120;
  st->gq_kps = 128;
  st->vkps = 128;
  st->vtok_work = 5120;
  st->spin_ticks = SPIN_TICKS;
  // Plain launches by default: one workgroup per CU is all that fits (LDS), the grid is one per
  // CU, and on a device not shared with concurrent work every workgroup is resident at once. A
  // plain launch starts right after the previous one on the stream; a cooperative launch, which
  // guarantees residency, starts about 20 us later. Should a workgroup ever not be resident,
  // the bounded waits end the launch with FL_E_TIMEOUT instead of hanging.
  st->coop = 0;
  if (const char* e = getenv("FLINT_AMD_COOPERATIVE")) st->coop = atoi(e) != 0;
  if (const char* e = getenv("FLINT_AMD_ATT_STEPS")) {  // tuning knob: steps per wave per slice
    const int v = atoi(e);
    if (v >= 1 && v <= 64) st->att_spw = v;
  }
  if (const char* e = getenv("FLINT_AMD_ATT_SLICES")) {  // tuning knob: a fixed key-slice count
    const int v = atoi(e);
    if (v >= 1 && v <= MAX_SLICES) st->att_spw = -v;
  }
  if (const char* e = getenv("FLINT_AMD_DEFER_SLICES")) {  // tuning knob: slices from which slice 0
    const int v = atoi(e);                                  // merges in the O phase
    if (v >= 2) st->defer_min = v;
  }
  if (const char* e = getenv("FLINT_AMD_GQA_MIN")) st->gq_min = std::max(0, atoi(e));  // tuning knob
  if (const char* e = getenv("FLINT_AMD_GQA_KEYS")) {  // tuning knob: keys per GQA slice
    const int v = atoi(e);
    if (v >= 16 && v <= 65536) st->gq_kps = v;
  }
  if (const char* e = getenv("FLINT_AMD_VERIFY_SLICE_KEYS")) {  // tuning knob: keys per verify slice
    const int v = atoi(e);
    if (v >= 16 && v <= 65536) st->vkps = v & ~15;
  }
  if (const char* e = getenv("FLINT_AMD_VERIFY_TOKEN_WORK")) {  // tuning knob (0: always by slices)
    const int v = atoi(e);
    if (v >= 0) st->vtok_work = v;
  }
  // speculative verify: its dynamic LDS (token rows staged for the matrix cores) must fit, and a
  // full grid of it must be co-resident
  st->verify_ok = 0;
  // (one attention unit per workgroup: at least one per query head; one ready flag per head)
  if (D <= 4096 && 2 * F / 16 <= VF_WORDS - VF_ACT && d->n_head <= cu && d->n_head <= VF_ACT - VF_ATTN) {
    const size_t vl = verify_lds_bytes(D);
    st->verify_ok = 1;
    for (const void* kv : {reinterpret_cast<const void*>(k_verify<1>), reinterpret_cast<const void*>(k_verify<2>)}) {
      int vocc = 0;
      if (!(hipFuncSetAttribute(kv, hipFuncAttributeMaxDynamicSharedMemorySize, (int)vl) == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&vocc, kv, NT, vl) == hipSuccess && vocc >= 1))
        st->verify_ok = 0;
    }
    (void)hipGetLastError();
  }
  int rc = FL_OK;
  if (rc == FL_OK) rc = uc_alloc(st, &st->h, (size_t)D * FL_MAX_VERIFY);
  if (rc == FL_OK) rc = uc_alloc(st, &st->qkv, (size_t)(NQKV / 2) * FL_MAX_VERIFY);
  if (rc == FL_OK) rc = uc_alloc(st, &st->attn, (size_t)D * FL_MAX_VERIFY);
  if (rc == FL_OK) rc = uc_alloc(st, &st->act, (size_t)F * FL_MAX_VERIFY);
  {
    // decode: attention slice partials; verify: down-projection part sums [D/16][KP][FL_MAX_VERIFY][16]
    const int gpp = std::max(1, std::min(NWAVE, D >> 7)), kp = ((F >> 7) + gpp - 1) / gpp;
    const size_t dec = (size_t)d->n_head * MAX_SLICES * 66, ver = (size_t)(D / 16) * kp * FL_MAX_VERIFY * 16;
    if (rc == FL_OK) rc = uc_alloc(st, &st->part, std::max(dec, ver));
  }
  if (rc == FL_OK) rc = uc_alloc(st, &st->vrows, (size_t)FL_MAX_VERIFY * (2 * D + F));
  if (rc == FL_OK) rc = uc_alloc(st, &st->vflag, (size_t)VF_WORDS);
  if (rc == FL_OK && st->verify_ok)
    rc = uc_alloc(st, &st->vpart, (size_t)d->n_head * VNS * FL_MAX_VERIFY * 66);
  if (rc == FL_OK) rc = uc_alloc(st, &st->shist, (size_t)G * 256);
  if (rc == FL_OK) rc = uc_alloc(st, &st->sword, (size_t)256 + 2 * G);
  if (rc == FL_OK) rc = dev_alloc(st, &st->amax, FL_MAX_VERIFY);
  if (rc == FL_OK) rc = dev_alloc(st, &st->done, 1);
  if (rc == FL_OK) rc = dev_alloc(st, &st->err, 1);
  if (rc == FL_OK) rc = dev_alloc(st, &st->stall, 1);
  if (rc != FL_OK) {
    fl_state_destroy(st);
    return rc;
  }
  *out = st;
  return FL_OK;
}

int fl_state_destroy(fl_state* st) {
  if (!st) return FL_E_ARG;
  hipDeviceSynchronize();
  for (int i = 0; i < st->nblocks; ++i) hipFree(st->blocks[i]);
  for (int i = 0; i < st->nuc; ++i) uc_release(st->uc[i]);  // never freed, reused
  free(st);
  return FL_OK;
}

int fl_state_reset(fl_state* st, void* stream) {
  if (!st) return FL_E_ARG;
  hipStream_t s = as_stream(stream);
  if (hipMemsetAsync(st->amax, 0, sizeof(unsigned long long) * FL_MAX_VERIFY, s) != hipSuccess)
    return FL_E_HIP;
  if (hipMemsetAsync(st->done, 0, sizeof(uint32_t), s) != hipSuccess) return FL_E_HIP;
  if (hipMemsetAsync(st->err, 0, sizeof(int32_t), s) != hipSuccess) return FL_E_HIP;
  return clear_exchange(st, s);
}

int fl_state_profile(fl_state* st, uint64_t* buf, int32_t slots_per_wg, int32_t* grid) {
  if (!st || (buf && slots_per_wg <= 0)) return FL_E_ARG;
  st->prof = reinterpret_cast<unsigned long long*>(buf);
  st->prof_slots = buf ? slots_per_wg : 0;
  if (grid) *grid = st->grid;
  return FL_OK;
}

int fl_state_buffers(fl_state* st, uint16_t** h, uint16_t** qkv, uint16_t** attn, uint16_t** act) {
  if (!st) return FL_E_ARG;
  if (h) *h = reinterpret_cast<uint16_t*>(st->h);
  if (qkv) *qkv = reinterpret_cast<uint16_t*>(st->qkv);
  if (attn) *attn = reinterpret_cast<uint16_t*>(st->attn);
  if (act) *act = reinterpret_cast<uint16_t*>(st->act);
  return FL_OK;
}

int fl_state_set_wait_limit(fl_state* st, uint64_t ticks) {
  if (!st) return FL_E_ARG;
  st->spin_ticks = ticks ? (unsigned long long)ticks : SPIN_TICKS;
  return FL_OK;
}

int fl_state_force_timeout(fl_state* st, int32_t on) {
  if (!st) return FL_E_ARG;
  st->force_timeout = on != 0;
  return FL_OK;
}

int fl_state_check(fl_state* st, void* stream) {
  if (!st) return FL_E_ARG;
  int32_t e = 0;
  if (hipStreamSynchronize(as_stream(stream)) != hipSuccess) return FL_E_HIP;
  if (hipMemcpy(&e, st->err, sizeof(e), hipMemcpyDeviceToHost) != hipSuccess) return FL_E_HIP;
  return e;
}

int fl_kv_move(fl_state* st, const int32_t* src, const int32_t* dst, int32_t n, void* stream) {
  if (!st || n < 0 || n > FL_MAX_VERIFY || (n > 0 && (!src || !dst))) return FL_E_ARG;
  KvMove mv{};
  mv.n = n;
  for (int i = 0; i < n; ++i) {
    if (src[i] < 0 || src[i] >= st->max_seq || dst[i] < 0 || dst[i] >= st->max_seq) return FL_E_POS;
    mv.src[i] = src[i];
    mv.dst[i] = dst[i];
  }
  if (n == 0) return FL_OK;
  hipLaunchKernelGGL(k_kv_move, dim3(st->d.n_layer * st->d.n_kv_head), dim3(KV_MOVE_THREADS), 0,
                     as_stream(stream), st->kc, st->vc, st->max_seq, mv);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}


int fl_decode_step(const fl_weights* w, fl_state* st, const int32_t* token_in, int32_t pos,
                   int32_t* token_out, float* logits, uint16_t* feat, void* stream) {
  if (!st || !token_in || !token_out || !weights_ok(w)) return FL_E_ARG;
  return decode_launch(w, st, token_in, nullptr, pos, token_out, logits, feat, stream);
}

int fl_decode_hidden(const fl_weights* w, fl_state* st, uint16_t* h, int32_t pos,
                     int32_t* token_out, float* logits, uint16_t* feat, void* stream) {
  if (!st || !h || !weights_ok(w)) return FL_E_ARG;
  return decode_launch(w, st, nullptr, h, pos, token_out, logits, feat, stream);
}

int fl_decode_sample(const fl_weights* w, fl_state* st, const int32_t* token_in, int32_t pos,
                     float temperature, int32_t top_k, uint64_t seed, uint64_t offset,
                     int32_t* token_out, float* logits, uint16_t* feat, void* stream) {
  if (!st || !token_in || !token_out || !weights_ok(w) || top_k < 0) return FL_E_ARG;
  if (!(temperature == temperature) || st->d.vocab > 65536) return FL_E_ARG;
  // one LM-head row per thread of a workgroup in the sampling epilogue
  {
    int R = (st->d.vocab + st->grid - 1) / st->grid;
    R += (R & 1);
    if (R > NT) return FL_E_ARG;
  }
  const float tdiv = temperature > 1e-5f ? temperature : 1e-5f;
  return decode_launch(w, st, token_in, nullptr, pos, token_out, logits, feat, stream,
                       SampleArgs{tdiv, top_k, seed, offset});
}

int fl_verify(const fl_weights* w, fl_state* st, const int32_t* tokens, int32_t m,
              const int32_t* depth, const uint8_t* amask, int32_t pos, int32_t* tokens_out,
              float* logits, uint16_t* feat, void* stream) {
  if (!st || !tokens || !depth || !amask || !tokens_out || !weights_ok(w)) return FL_E_ARG;
  if (!w->wqkv_t || !w->wo_t || !w->wgu_t || !w->wd_t) return FL_E_ARG;  // verify reads the tiled copies
  if (m < 1 || m > FL_MAX_VERIFY) return FL_E_M;
  if (pos < 0 || pos + m > st->max_seq) return FL_E_POS;
  if (!st->verify_ok) return FL_E_ARG;
  // the down projection splits K into parts of 8 groups, each needing a workgroup of its own,
  // and each 16-row tile of h has an owning workgroup that keeps its rows in LDS
  {
    const int gpp = std::min(NWAVE, st->d.dim >> 7);
    if (st->vgrid < ((st->d.inter >> 7) + gpp - 1) / gpp || st->vgrid < st->d.dim / 16) return FL_E_ARG;
  }
  if (maybe_clear(st, as_stream(stream)) != FL_OK) return FL_E_LAUNCH;
  DecodeParams p = base_params(w, st, pos);
  p.M = m;
  p.tokens = tokens;
  p.depth = depth;
  p.amask = amask;
  p.tokens_out = tokens_out;
  p.logits = logits;
  p.feat = feat;
  p.prof = st->prof;
  p.prof_slots = st->prof_slots;
  void* args[] = {&p};
  const unsigned lds = (unsigned)verify_lds_bytes(st->d.dim);
  const void* kv = verify_by_tokens(st->d.n_head, m, pos, st->vgrid, st->vtok_work)
                       ? reinterpret_cast<const void*>(k_verify<1>)
                       : reinterpret_cast<const void*>(k_verify<2>);
  const hipError_t e =
      st->coop ? hipLaunchCooperativeKernel(kv, dim3(st->vgrid), dim3(NT), args, lds, as_stream(stream))
               : hipLaunchKernel(kv, dim3(st->vgrid), dim3(NT), args, lds, as_stream(stream));
  if (e != hipSuccess) return FL_E_LAUNCH;
  advance_epoch(st);
  return FL_OK;
}

}  // extern "C"
