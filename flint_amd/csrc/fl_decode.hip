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
//  * the next phase's weight chunks are loaded into registers BEFORE the grid barrier, so the
//    HBM stream overlaps the barrier latency and the epilogue;
//  * RMSNorm is recomputed by every workgroup from the residual (no barrier of its own);
//    RoPE + KV append are fused into the QKV epilogue (NEOX pairs live in adjacent packed rows);
//    SwiGLU is fused into the gate/up epilogue (gate/up rows interleaved); residual adds are fused
//    into the O / down epilogues; greedy argmax is fused into the LM head;
//  * attention is flash-decode over (kv-group, 64-key chunk) units, one wave each, all query heads
//    of a GQA group sharing every K/V load; the last unit of a group to finish merges the group's
//    partials (arrival counter), so attention costs a single grid barrier;
//  * 5 grid barriers per layer, each a single agent-scope counter with a bounded spin.
#include "fl_common.h"
#include <stdlib.h>
#include <string.h>

namespace {

constexpr int NT = 512;              // threads per workgroup
constexpr int NWAVE = NT / FL_WAVE;  // waves per workgroup
constexpr int MAXC = 12;             // max 16-byte weight chunks per thread in one GEMV phase
constexpr int XS_MAX = 8192;         // max staged activation length (bf16 elements)
constexpr int ROWS_MAX = 256;        // max rows per workgroup in one GEMV phase
constexpr int QPG_MAX = 8;           // max query heads per kv group
constexpr int KC = 64;               // keys per attention unit (one per lane)
constexpr int LM_MAXC = 8;           // max 16-byte chunks per lane of one LM-head row (D <= 4096)
constexpr int LM_RB = 2;             // LM-head rows per wave per batch
constexpr unsigned long long SPIN_TICKS = 200000000ull;  // 2 s of the 100 MHz realtime clock
// LDS float workspace: GEMV per-chunk partials, or per-wave attention q/p tiles
constexpr int WS_FLOATS = (MAXC * NT > NWAVE * 2 * QPG_MAX * 64) ? MAXC * NT : NWAVE * 2 * QPG_MAX * 64;

struct DecodeParams {
  fl_weights w;
  uint16_t *kc, *vc;        // [NL, NKV, S, 64]
  uint16_t *h, *q, *attn, *act;
  float* part;              // attention partials
  uint32_t* cnt;            // [NKV] attention arrivals
  unsigned long long* bar;  // grid barrier counter
  unsigned long long* amax; // argmax key
  uint32_t* done;           // final arrivals
  int32_t* err;             // abort flag (barrier timeout)
  const int32_t* token_in;
  int32_t* token_out;
  float* logits;
  uint16_t* feat;
  int D, NH, NKV, F, V, NL, S, pos;
  float eps, emb_mult, attn_scale, resid_mult, logits_scaling;
  unsigned long long bar_base;
};

__device__ __forceinline__ void row_range(int n, int wg, int G, int& r0, int& rows) {
  int R = (n + G - 1) / G;
  R += (R & 1);
  r0 = wg * R;
  rows = min(R, n - r0);
  if (rows < 0) rows = 0;
}

// Grid barrier: one agent-scope counter, monotonic across launches (the host keeps the base).
__device__ void grid_sync(const DecodeParams& p, unsigned long long& target) {
  target += gridDim.x;
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(p.bar, 1ull, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    if (__hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
      const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
      unsigned it = 0;
      while (__hip_atomic_load(p.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        __builtin_amdgcn_s_sleep(1);
        if ((++it & 255u) == 0) {
          if (__builtin_amdgcn_s_memrealtime() - t0 > SPIN_TICKS) {
            __hip_atomic_store(p.err, (int32_t)FL_E_TIMEOUT, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          if (__hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// xs = RMSNorm(src) with gpt-fast's rounding (engine/model.py:231-242):
//   n = bf16(x * rsqrt(mean(x^2) + eps)) ; out = bf16(n * w)
// When use_mult, src is an embedding row and x = bf16(src * mult) (engine/model.py:138).
__device__ void wg_norm(const uint16_t* __restrict__ src, bool use_mult, float mult,
                        const uint16_t* __restrict__ nw, int D, float eps, uint16_t* xs,
                        float* red) {
  const int tid = threadIdx.x;
  float ss = 0.0f;
  for (int i = tid; i < (D >> 3); i += NT) {
    const uint4 v = reinterpret_cast<const uint4*>(src)[i];
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a = bflo(in[j]), b = bfhi(in[j]);
      if (use_mult) {
        a = rbf(a * mult);
        b = rbf(b * mult);
      }
      ss += a * a;
      ss += b * b;
      o[j] = pack_bf16x2(a, b);
    }
    reinterpret_cast<uint4*>(xs)[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) tot += red[w];
  const float r = 1.0f / sqrtf(tot / (float)D + eps);
  for (int i = tid; i < (D >> 3); i += NT) {
    const uint4 v = reinterpret_cast<const uint4*>(xs)[i];
    const uint4 g = reinterpret_cast<const uint4*>(nw)[i];
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float na = rbf(bflo(in[j]) * r), nb = rbf(bfhi(in[j]) * r);
      o[j] = pack_bf16x2(na * bflo(gw[j]), nb * bfhi(gw[j]));
    }
    reinterpret_cast<uint4*>(xs)[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  __syncthreads();
}

// xs = src (bf16 vector of length n, n % 8 == 0)
__device__ __forceinline__ void wg_stage(const uint16_t* __restrict__ src, int n, uint16_t* xs) {
  for (int i = threadIdx.x; i < (n >> 3); i += NT)
    reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(src)[i];
  __syncthreads();
}

// Issue this workgroup's weight chunks for rows [r0, r0+rows) of a [N, K] int4 matrix.
__device__ __forceinline__ void gemv_load(const uint32_t* __restrict__ q,
                                          const uint32_t* __restrict__ sz, int r0, int rows, int K,
                                          uint4 (&wr)[MAXC], uint32_t (&sr)[MAXC]) {
  const int total = rows * (K >> 5);
  const uint4* wb = reinterpret_cast<const uint4*>(q + (size_t)r0 * (K >> 3));
  const uint32_t* sb = sz + (size_t)r0 * (K >> 7);
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int f = threadIdx.x + i * NT;
    if (f < total) {
      wr[i] = wb[f];
      sr[i] = sb[f >> 2];
    }
  }
}

// rs[r] = sum_k x[k] * dq[r0+r, k] for the chunks loaded by gemv_load; x staged in xs.
__device__ __forceinline__ void gemv_compute(const uint4 (&wr)[MAXC], const uint32_t (&sr)[MAXC],
                                             int rows, int K, const uint16_t* xs, float* part,
                                             float* rs) {
  const int tid = threadIdx.x;
  const int cpr = K >> 5;
  const int total = rows * cpr;
  int c = tid % cpr;
  const int step = NT % cpr;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int f = tid + i * NT;
    if (f < total)
      part[f] = chunk_dot(wr[i], sr[i], reinterpret_cast<const uint4*>(xs + c * 32), 0.0f);
    c += step;
    if (c >= cpr) c -= cpr;
    __builtin_amdgcn_sched_barrier(0);  // keep one chunk's temporaries live at a time
  }
  __syncthreads();
  int L = 64;
  while (L * rows > NT) L >>= 1;
  const int row = tid / L, li = tid % L;
  float acc = 0.0f;
  if (row < rows)
    for (int j = li; j < cpr; j += L) acc += part[row * cpr + j];
  acc = group_sum(acc, L);
  if (row < rows && li == 0) rs[row] = acc;
  __syncthreads();
}

template <int QPG>
__device__ void attention_phase(const DecodeParams& p, int l, float* wl) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = gridDim.x;
  const int T = p.pos + 1;
  const int nch = (T + KC - 1) / KC;
  const int units = p.NKV * nch;
  float* qs = wl + wave * (2 * QPG_MAX * 64);
  float* ps = qs + QPG_MAX * 64;
  for (int u = wave * G + blockIdx.x; u < units; u += G * NWAVE) {
    const int g = u / nch, ch = u - g * nch, t0 = ch * KC;
    const size_t cbase = (size_t)(l * p.NKV + g) * p.S * 64;
    const uint16_t* kb = p.kc + cbase;
    const uint16_t* vb = p.vc + cbase;
    for (int i = lane; i < QPG * 64; i += 64) qs[i] = bf2f(p.q[g * QPG * 64 + i]);
    wave_sync();
    // scores: lane = key
    const int t = t0 + lane;
    const bool valid = t < T;
    float s[QPG];
#pragma unroll
    for (int h = 0; h < QPG; ++h) s[h] = 0.0f;
    if (valid) {
      const uint4* kr = reinterpret_cast<const uint4*>(kb + (size_t)t * 64);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const uint4 kv = kr[jj];
        const float kf[8] = {bflo(kv.x), bfhi(kv.x), bflo(kv.y), bfhi(kv.y),
                             bflo(kv.z), bfhi(kv.z), bflo(kv.w), bfhi(kv.w)};
#pragma unroll
        for (int h = 0; h < QPG; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) s[h] = __builtin_fmaf(qs[h * 64 + jj * 8 + e], kf[e], s[h]);
      }
    }
    float mh[QPG], lh[QPG];
#pragma unroll
    for (int h = 0; h < QPG; ++h) {
      const float sv = valid ? s[h] * p.attn_scale : -INFINITY;
      const float m = wave_max(sv);
      const float pv = valid ? expf(sv - m) : 0.0f;
      lh[h] = wave_sum(pv);
      mh[h] = m;
      ps[h * 64 + lane] = pv;
    }
    wave_sync();
    // P.V: lane = (4-dim slice j4, key lane group kg of 4)
    const int j4 = lane & 15, kg = lane >> 4;
    float acc[QPG][4];
#pragma unroll
    for (int h = 0; h < QPG; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[h][e] = 0.0f;
#pragma unroll 4
    for (int kk = 0; kk < KC / 4; ++kk) {
      const int tt = kg + 4 * kk;
      if (t0 + tt < T) {
        const uint2 vv = *reinterpret_cast<const uint2*>(vb + (size_t)(t0 + tt) * 64 + j4 * 4);
        const float vf[4] = {bflo(vv.x), bfhi(vv.x), bflo(vv.y), bfhi(vv.y)};
#pragma unroll
        for (int h = 0; h < QPG; ++h) {
          const float pw = ps[h * 64 + tt];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[h][e] = __builtin_fmaf(pw, vf[e], acc[h][e]);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < QPG; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[h][e];
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        acc[h][e] = v;
      }
    float* pp = p.part + (size_t)u * QPG * 66;
    if (kg == 0) {
#pragma unroll
      for (int h = 0; h < QPG; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) pp[h * 66 + 2 + j4 * 4 + e] = acc[h][e];
    }
    if (lane == 0) {
#pragma unroll
      for (int h = 0; h < QPG; ++h) {
        pp[h * 66] = mh[h];
        pp[h * 66 + 1] = lh[h];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    uint32_t old = 0;
    if (lane == 0)
      old = __hip_atomic_fetch_add(p.cnt + g, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0, 64);
    if (old == (uint32_t)(nch - 1)) {
      // last unit of group g: merge the nch partials (log-sum-exp rescale), fixed order
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      const float* gp = p.part + (size_t)g * nch * QPG * 66;
      for (int h = 0; h < QPG; ++h) {
        float M = -INFINITY;
        for (int c = 0; c < nch; ++c) M = fmaxf(M, gp[(size_t)(c * QPG + h) * 66]);
        float Ls = 0.0f, O = 0.0f;
        for (int c = 0; c < nch; ++c) {
          const float* cp = gp + (size_t)(c * QPG + h) * 66;
          const float e = expf(cp[0] - M);
          Ls += cp[1] * e;
          O += cp[2 + lane] * e;
        }
        p.attn[(g * QPG + h) * 64 + lane] = (uint16_t)f2bf(O / Ls);
      }
      if (lane == 0) __hip_atomic_store(p.cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    wave_sync();
  }
}

template <int QPG>
__global__ __launch_bounds__(NT, 1) void k_decode(DecodeParams p) {
  __shared__ __align__(16) uint16_t xs[XS_MAX];
  __shared__ __align__(16) float part[WS_FLOATS];
  __shared__ float rs[ROWS_MAX];
  __shared__ float red[64];
  __shared__ unsigned long long kred[NWAVE];

  const int tid = threadIdx.x, wg = blockIdx.x, G = gridDim.x;
  const int D = p.D, F = p.F, NKV = p.NKV, NH = p.NH;
  const int NQKV = (NH + 2 * NKV) * 64;
  const int pos = p.pos;
  unsigned long long target = p.bar_base;
  int token = *p.token_in;
  if (token < 0 || token >= p.V) {  // bad device-side token: record it, read row 0 (no fault)
    if (tid == 0 && wg == 0)
      __hip_atomic_store(p.err, (int32_t)FL_E_ARG, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    token = 0;
  }
  const uint16_t* erow = p.w.embed + (size_t)token * D;

  int r0d, rowsd;  // this workgroup's rows of every [D]-output GEMV (O, down): it owns h there
  row_range(D, wg, G, r0d, rowsd);
  // h = bf16(embed[token] * emb_mult) on the owned rows (engine/model.py:138)
  for (int i = tid; i < rowsd; i += NT)
    p.h[r0d + i] = (uint16_t)f2bf(bf2f(erow[r0d + i]) * p.emb_mult);

  uint4 wr[MAXC];
  uint32_t sr[MAXC];
  int r0, rows;
  row_range(NQKV, wg, G, r0, rows);
  gemv_load(p.w.wqkv_q, p.w.wqkv_sz, r0, rows, D, wr, sr);

  for (int l = 0; l < p.NL; ++l) {
    // ---------------- P1: RMSNorm + QKV + RoPE + KV append ----------------
    if (l == 0)
      wg_norm(erow, true, p.emb_mult, p.w.attn_norm, D, p.eps, xs, red);
    else
      wg_norm(p.h, false, 1.0f, p.w.attn_norm + (size_t)l * D, D, p.eps, xs, red);
    row_range(NQKV, wg, G, r0, rows);
    gemv_compute(wr, sr, rows, D, xs, part, rs);
    if (tid < (rows >> 1)) {
      const int srow = r0 + 2 * tid;
      const int hh = srow >> 6, j = (srow & 63) >> 1;
      const float a = rbf(rs[2 * tid]), b = rbf(rs[2 * tid + 1]);
      float oa = a, ob = b;
      if (hh < NH + NKV) {  // RoPE (engine/model.py:257-269 on NEOX pairs j, j+32)
        const uint32_t cs = reinterpret_cast<const uint32_t*>(p.w.rope)[pos * 32 + j];
        const float c = bflo(cs), sn = bfhi(cs);
        oa = rbf(a * c - b * sn);
        ob = rbf(b * c + a * sn);
      }
      if (hh < NH) {
        p.q[hh * 64 + j] = (uint16_t)f2bf(oa);
        p.q[hh * 64 + j + 32] = (uint16_t)f2bf(ob);
      } else {
        const int g = (hh < NH + NKV) ? hh - NH : hh - NH - NKV;
        uint16_t* dst = ((hh < NH + NKV) ? p.kc : p.vc) +
                        ((size_t)(l * NKV + g) * p.S + pos) * 64;
        dst[j] = (uint16_t)f2bf(oa);
        dst[j + 32] = (uint16_t)f2bf(ob);
      }
    }
    __syncthreads();
    row_range(D, wg, G, r0, rows);
    gemv_load(p.w.wo_q + (size_t)l * D * (D >> 3), p.w.wo_sz + (size_t)l * D * (D >> 7), r0, rows,
              D, wr, sr);
    grid_sync(p, target);

    // ---------------- P2: GQA flash-decode attention ----------------
    attention_phase<QPG>(p, l, part);
    grid_sync(p, target);

    // ---------------- P3: O projection + residual ----------------
    wg_stage(p.attn, D, xs);
    row_range(D, wg, G, r0, rows);
    gemv_compute(wr, sr, rows, D, xs, part, rs);
    if (tid < rows) {  // h = bf16(h + bf16(bf16(o) * rm))  (engine/model.py:162)
      const int r = r0 + tid;
      const float o = rbf(rbf(rs[tid]) * p.resid_mult);
      p.h[r] = (uint16_t)f2bf(bf2f(p.h[r]) + o);
    }
    __syncthreads();
    row_range(2 * F, wg, G, r0, rows);
    gemv_load(p.w.wgu_q + (size_t)l * 2 * F * (D >> 3), p.w.wgu_sz + (size_t)l * 2 * F * (D >> 7),
              r0, rows, D, wr, sr);
    grid_sync(p, target);

    // ---------------- P4: RMSNorm + gate/up + SwiGLU ----------------
    wg_norm(p.h, false, 1.0f, p.w.ffn_norm + (size_t)l * D, D, p.eps, xs, red);
    row_range(2 * F, wg, G, r0, rows);
    gemv_compute(wr, sr, rows, D, xs, part, rs);
    if (tid < (rows >> 1)) {  // act = bf16(bf16(silu(g)) * u)  (engine/model.py:227-228)
      const float g = rbf(rs[2 * tid]), u = rbf(rs[2 * tid + 1]);
      p.act[(r0 >> 1) + tid] = (uint16_t)f2bf(rbf(silu_f(g)) * u);
    }
    __syncthreads();
    row_range(D, wg, G, r0, rows);
    gemv_load(p.w.wd_q + (size_t)l * D * (F >> 3), p.w.wd_sz + (size_t)l * D * (F >> 7), r0, rows,
              F, wr, sr);
    grid_sync(p, target);

    // ---------------- P5: down projection + residual ----------------
    wg_stage(p.act, F, xs);
    row_range(D, wg, G, r0, rows);
    gemv_compute(wr, sr, rows, F, xs, part, rs);
    if (tid < rows) {  // out = bf16(h + bf16(bf16(d) * rm))  (engine/model.py:163)
      const int r = r0 + tid;
      const float o = rbf(rbf(rs[tid]) * p.resid_mult);
      p.h[r] = (uint16_t)f2bf(bf2f(p.h[r]) + o);
    }
    __syncthreads();
    if (l + 1 < p.NL) {
      row_range(NQKV, wg, G, r0, rows);
      gemv_load(p.w.wqkv_q + (size_t)(l + 1) * NQKV * (D >> 3),
                p.w.wqkv_sz + (size_t)(l + 1) * NQKV * (D >> 7), r0, rows, D, wr, sr);
    }
    grid_sync(p, target);
  }

  // ---------------- final norm + tied bf16 LM head + greedy argmax ----------------
  wg_norm(p.h, false, 1.0f, p.w.final_norm, D, p.eps, xs, red);
  if (p.feat && wg == 0)
    for (int i = tid; i < D; i += NT) p.feat[i] = xs[i];
  const int lane = tid & 63, wave = tid >> 6;
  row_range(p.V, wg, G, r0, rows);
  const int nck = D >> 3;  // 16-byte chunks per row
  unsigned long long best = 0ull;
  for (int rb = wave * LM_RB; rb < rows; rb += NWAVE * LM_RB) {
    uint4 ev[LM_RB][LM_MAXC];
#pragma unroll
    for (int rr = 0; rr < LM_RB; ++rr) {
      const uint4* er = reinterpret_cast<const uint4*>(p.w.embed + (size_t)(r0 + rb + rr) * D);
#pragma unroll
      for (int i = 0; i < LM_MAXC; ++i) {
        const int c = lane + 64 * i;
        if (rb + rr < rows && c < nck) ev[rr][i] = er[c];
      }
    }
#pragma unroll
    for (int rr = 0; rr < LM_RB; ++rr) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < LM_MAXC; ++i) {
        const int c = lane + 64 * i;
        if (rb + rr < rows && c < nck) {
          const uint4 xv = reinterpret_cast<const uint4*>(xs)[c];
          acc = dot2_bf16(ev[rr][i].x, xv.x, acc);
          acc = dot2_bf16(ev[rr][i].y, xv.y, acc);
          acc = dot2_bf16(ev[rr][i].z, xv.z, acc);
          acc = dot2_bf16(ev[rr][i].w, xv.w, acc);
        }
      }
      acc = wave_sum(acc);
      acc = __shfl(acc, 0, 64);
      if (rb + rr < rows) {
        const int r = r0 + rb + rr;
        // logits = bf16(bf16(x . E^T) / logits_scaling)  (engine/model.py:144)
        const float lg = rbf(rbf(acc) / p.logits_scaling);
        if (p.logits && lane == 0) p.logits[r] = lg;
        best = u64max(best, amax_key(lg, (uint32_t)r));
      }
    }
  }
  if (lane == 0) kred[wave] = best;
  __syncthreads();
  if (tid == 0) {
    unsigned long long b = kred[0];
    for (int w = 1; w < NWAVE; ++w) b = u64max(b, kred[w]);
    __hip_atomic_fetch_max(p.amax, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t old = __hip_atomic_fetch_add(p.done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (uint32_t)(G - 1)) {
      const unsigned long long fin = __hip_atomic_load(p.amax, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *p.token_out = (int32_t)amax_index(fin);
      __hip_atomic_store(p.amax, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

typedef void (*decode_fn)(DecodeParams);

decode_fn pick_decode(int qpg) {
  switch (qpg) {
    case 1: return k_decode<1>;
    case 2: return k_decode<2>;
    case 4: return k_decode<4>;
    case 5: return k_decode<5>;
    case 8: return k_decode<8>;
    default: return nullptr;
  }
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

int phase_fits(int n, int k, int G) {
  int R = (n + G - 1) / G;
  R += (R & 1);
  return R <= ROWS_MAX && (long)R * (k >> 5) <= (long)MAXC * NT;
}

}  // namespace

struct fl_state {
  fl_model_desc d;
  int max_seq;
  int grid;
  int qpg;
  int nbar;  // grid barriers per decode launch
  uint16_t *kc, *vc;
  uint16_t *h, *q, *attn, *act;
  float* part;
  uint32_t* cnt;
  unsigned long long* bar;
  unsigned long long* amax;
  uint32_t* done;
  int32_t* err;
  unsigned long long bar_base;
  void* blocks[8];
  int nblocks;
};

namespace {
template <typename T>
int dev_alloc(fl_state* st, T** p, size_t count) {
  void* v = nullptr;
  if (hipMalloc(&v, count * sizeof(T) + 256) != hipSuccess) return FL_E_HIP;
  if (hipMemset(v, 0, count * sizeof(T) + 256) != hipSuccess) return FL_E_HIP;
  st->blocks[st->nblocks++] = v;
  *p = reinterpret_cast<T*>(v);
  return FL_OK;
}
}  // namespace

extern "C" {

int fl_device_info(int32_t* num_cu, int32_t* decode_grid) {
  int dev = 0, cu = 0, occ = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FL_E_HIP;
  if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return FL_E_HIP;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(k_decode<5>),
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
  const int qpg = d->n_head / d->n_kv_head;
  if (!pick_decode(qpg) || qpg > QPG_MAX) return FL_E_ARG;
  int dev = 0, cu = 0, occ = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FL_E_HIP;
  if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return FL_E_HIP;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &occ, reinterpret_cast<const void*>(pick_decode(qpg)), NT, 0) != hipSuccess)
    return FL_E_HIP;
  if (occ < 1 || cu < 1) return FL_E_LAUNCH;
  const int G = cu;
  const int D = d->dim, F = d->inter, NQKV = (d->n_head + 2 * d->n_kv_head) * FL_HEAD_DIM;
  if (!phase_fits(NQKV, D, G) || !phase_fits(D, D, G) || !phase_fits(2 * F, D, G) ||
      !phase_fits(D, F, G))
    return FL_E_ARG;
  fl_state* st = (fl_state*)calloc(1, sizeof(fl_state));
  if (!st) return FL_E_HIP;
  st->d = *d;
  st->max_seq = max_seq;
  st->grid = G;
  st->qpg = qpg;
  st->nbar = 5 * d->n_layer;
  st->kc = k_cache;
  st->vc = v_cache;
  const int nch_max = (max_seq + FL_MAX_VERIFY + KC - 1) / KC;
  int rc = FL_OK;
  if (rc == FL_OK) rc = dev_alloc(st, &st->h, (size_t)D * FL_MAX_VERIFY);
  if (rc == FL_OK) rc = dev_alloc(st, &st->q, (size_t)NQKV * FL_MAX_VERIFY);
  if (rc == FL_OK) rc = dev_alloc(st, &st->attn, (size_t)D * FL_MAX_VERIFY);
  if (rc == FL_OK) rc = dev_alloc(st, &st->act, (size_t)F * FL_MAX_VERIFY);
  if (rc == FL_OK)
    rc = dev_alloc(st, &st->part, (size_t)d->n_kv_head * nch_max * QPG_MAX * 66 * FL_MAX_VERIFY);
  if (rc == FL_OK) rc = dev_alloc(st, &st->cnt, (size_t)d->n_kv_head * FL_MAX_VERIFY);
  if (rc == FL_OK) rc = dev_alloc(st, &st->bar, 1);
  if (rc == FL_OK) rc = dev_alloc(st, &st->amax, FL_MAX_VERIFY);
  if (rc == FL_OK) rc = dev_alloc(st, &st->done, 1);
  if (rc == FL_OK) rc = dev_alloc(st, &st->err, 1);
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
  free(st);
  return FL_OK;
}

int fl_state_reset(fl_state* st, void* stream) {
  if (!st) return FL_E_ARG;
  hipStream_t s = as_stream(stream);
  if (hipMemsetAsync(st->cnt, 0, sizeof(uint32_t) * st->d.n_kv_head * FL_MAX_VERIFY, s) != hipSuccess)
    return FL_E_HIP;
  if (hipMemsetAsync(st->amax, 0, sizeof(unsigned long long) * FL_MAX_VERIFY, s) != hipSuccess)
    return FL_E_HIP;
  if (hipMemsetAsync(st->done, 0, sizeof(uint32_t), s) != hipSuccess) return FL_E_HIP;
  if (hipMemsetAsync(st->err, 0, sizeof(int32_t), s) != hipSuccess) return FL_E_HIP;
  if (hipMemsetAsync(st->bar, 0, sizeof(unsigned long long), s) != hipSuccess) return FL_E_HIP;
  st->bar_base = 0;
  return FL_OK;
}

int fl_state_check(fl_state* st, void* stream) {
  if (!st) return FL_E_ARG;
  int32_t e = 0;
  if (hipStreamSynchronize(as_stream(stream)) != hipSuccess) return FL_E_HIP;
  if (hipMemcpy(&e, st->err, sizeof(e), hipMemcpyDeviceToHost) != hipSuccess) return FL_E_HIP;
  return e;
}

int fl_decode_step(const fl_weights* w, fl_state* st, const int32_t* token_in, int32_t pos,
                   int32_t* token_out, float* logits, uint16_t* feat, void* stream) {
  if (!w || !st || !token_in || !token_out) return FL_E_ARG;
  if (!w->wqkv_q || !w->wqkv_sz || !w->wo_q || !w->wo_sz || !w->wgu_q || !w->wgu_sz || !w->wd_q ||
      !w->wd_sz || !w->attn_norm || !w->ffn_norm || !w->final_norm || !w->embed || !w->rope)
    return FL_E_ARG;
  if (pos < 0 || pos >= st->max_seq || pos >= w->rope_len) return FL_E_POS;
  DecodeParams p;
  memset(&p, 0, sizeof(p));
  p.w = *w;
  p.kc = st->kc;
  p.vc = st->vc;
  p.h = st->h;
  p.q = st->q;
  p.attn = st->attn;
  p.act = st->act;
  p.part = st->part;
  p.cnt = st->cnt;
  p.bar = st->bar;
  p.amax = st->amax;
  p.done = st->done;
  p.err = st->err;
  p.token_in = token_in;
  p.token_out = token_out;
  p.logits = logits;
  p.feat = feat;
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
  p.bar_base = st->bar_base;
  void* args[] = {&p};
  const hipError_t e =
      hipLaunchCooperativeKernel(reinterpret_cast<const void*>(pick_decode(st->qpg)), dim3(st->grid),
                                 dim3(NT), args, 0, as_stream(stream));
  if (e != hipSuccess) return FL_E_LAUNCH;
  st->bar_base += (unsigned long long)st->nbar * st->grid;
  return FL_OK;
}

}  // extern "C"
