// Temperature / top-k sampling of logit rows on the GPU (reference engine/generate.py:36-55).
//
// Each row is split over up to SP_C chunks, one workgroup each, in one plain launch; per-row
// barriers (an arrival counter in the row's scratch, bounded waits) separate the steps that need
// the whole row. The reference's steps with its bf16 rounding
// points: x = bf16(l / max(T, 1e-5)); the top-k pivot is the k-th largest x, found by a two-pass
// radix select over the 16-bit ordered keys of the bf16 values (each chunk's 256-bin histogram
// of the high byte, summed over the row in a fixed order, then the low byte within the selected
// bin); x < pivot drops out; p = bf16(exp(x - max) / sum), the sum of the chunks' partial sums in
// chunk order; q = bf16(-log(u)) with u from Philox4x32-10 keyed by the caller's seed, or q
// given; the sample is the first index of the largest bf16(p / q), which is
// multinomial_sample_one_no_sync's argmax(probs / exponential noise): 64-bit atomicMax of
// (ratio, ~index) per row, read out by the row's last chunk to finish.
#include <algorithm>
#include <mutex>
#include <stdlib.h>
#include "fl_common.h"

namespace {

constexpr int SAMPLE_MAXV = 65536;            // vocab limit

constexpr int SP_NT = 256;                     // threads per chunk workgroup
constexpr int SP_C = 64;                       // chunks per row (at most)
constexpr int SP_PT = 4;                       // values per thread: chunk <= 1024, vocab <= 65536
constexpr int SP_NWAVE = SP_NT / FL_WAVE;

// per-row scratch of the cooperative sampler (device memory owned by the library)
struct SampleWs {
  int hist[SP_C][2][256];                      // per chunk: high-byte, low-byte key histograms
  float mx[SP_C], ps[SP_C];                    // per chunk: max x, partial sum of exp(x - max)
  unsigned long long best;                     // (ratio bits, ~index), atomicMax
  unsigned int arrived;                        // chunks done (the last one reads best out)
  unsigned int bar;                            // barrier arrivals of this launch (reset by the last chunk)
  unsigned int fail;                           // a chunk's barrier wait timed out (reset by the last chunk)
};

constexpr unsigned long long SAMPLE_WAIT_TICKS = 200000000ull;  // 2 s of the 100 MHz realtime clock

// scratch words written before a row barrier and read after it by other workgroups (possibly on
// other XCDs): device-coherent accesses
__device__ __forceinline__ void st_ws(unsigned* a, unsigned v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_ws(float* a, unsigned v) { st_ws(reinterpret_cast<unsigned*>(a), v); }
__device__ __forceinline__ unsigned ld_ws(unsigned* a) {
  return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Barrier of the C chunk workgroups of one row: every thread's scratch stores are acknowledged
// (s_waitcnt 0) before the workgroup's arrival is counted, and the workgroup leaves once the
// row's count reaches `target` (C per barrier so far). The launch is a plain one: its grid (at
// most 16 rows x 64 chunks of 256 threads) is checked on the host to fit the device at once, so
// every chunk is resident on an idle device; should one not be (other work holding its CU), the
// wait gives up after 2 s and the row's token is reported as -1 instead of hanging.
__device__ __forceinline__ void row_sync(SampleWs* ws, unsigned target, bool* timed_out) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(&ws->bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (ld_ws(&ws->bar) < target) {
      __builtin_amdgcn_s_sleep(2);
      if (__builtin_amdgcn_s_memrealtime() - t0 > SAMPLE_WAIT_TICKS) {
        *timed_out = true;
        break;
      }
    }
  }
  __syncthreads();
}

__device__ __forceinline__ float wg_max(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = red[0];
  for (int w = 1; w < SP_NWAVE; ++w) v = fmaxf(v, red[w]);
  return v;
}
__device__ __forceinline__ float wg_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = 0.0f;
  for (int w = 0; w < SP_NWAVE; ++w) v += red[w];
  return v;
}
__device__ __forceinline__ unsigned long long wg_umax(unsigned long long v, unsigned long long* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long w = (unsigned long long)__shfl_xor((long long)v, o, 64);
    v = w > v ? w : v;
  }
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = red[0];
  for (int w = 1; w < SP_NWAVE; ++w) v = red[w] > v ? red[w] : v;
  return v;
}

__global__ __launch_bounds__(SP_NT) void k_sample(const float* __restrict__ logits, int V, int C, int row0,
                                                  float tdiv, int top_k, uint32_t seed_lo,
                                                  uint32_t seed_hi, uint32_t off_lo, uint32_t off_hi,
                                                  const float* __restrict__ noise,
                                                  int32_t* __restrict__ tokens_out,
                                                  float* __restrict__ probs_out, SampleWs* __restrict__ wsa) {
  __shared__ int hist[256];
  __shared__ int sel[2];
  __shared__ float red[SP_NWAVE];
  __shared__ unsigned long long ured[SP_NWAVE];
  __shared__ bool last, timed_out;
  const int tid = threadIdx.x, row = blockIdx.x / C, c = blockIdx.x % C;
  const int CH = (V + C - 1) / C, j0 = c * CH, j1 = min(V, j0 + CH);
  SampleWs* ws = wsa + row;
  unsigned nsync = 0;  // row barriers passed
  if (tid == 0) timed_out = false;
  // the row's argmax word and arrival count start at zero: cleared here, before the first row
  // barrier, which orders it before every chunk's use after the last one. The barrier counter
  // itself is zero at launch: the last chunk of the previous call on this scratch reset it.
  if (c == 0 && tid == 0) {
    __hip_atomic_store(&ws->best, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&ws->arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const float* lg = logits + (size_t)row * V;
  float x[SP_PT];
  // x = bf16(bf16(logit) / max(T, 1e-5))  (generate.py:42); max over the chunk
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < SP_PT; ++e) {
    const int j = j0 + tid + e * SP_NT;
    x[e] = j < j1 ? rbf(rbf(lg[j]) / tdiv) : -INFINITY;
    mx = fmaxf(mx, x[e]);
  }
  mx = wg_max(mx, red);
  if (tid == 0) st_ws(&ws->mx[c], __float_as_uint(mx));
  // top-k pivot (generate.py:44-47): keys >= the k-th largest key stay
  uint32_t pivot = 0;
  const bool topk = top_k > 0 && top_k < V;
  if (topk) {
    int k = top_k;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      hist[tid] = 0;  // SP_NT == 256 bins
      __syncthreads();
#pragma unroll
      for (int e = 0; e < SP_PT; ++e) {
        const uint32_t key = bf_key(x[e]);
        const bool in = (j0 + tid + e * SP_NT < j1) & (pass == 0 || (key >> 8) == (pivot >> 8));
        if (in) atomicAdd(&hist[pass == 0 ? (key >> 8) : (key & 0xFFu)], 1);
      }
      __syncthreads();
      st_ws(reinterpret_cast<unsigned*>(&ws->hist[c][pass][tid]), (unsigned)hist[tid]);
      row_sync(ws, (unsigned)C * ++nsync, &timed_out);
      // the row's counts: thread t sums bins 4(t % 64) .. +3 over chunks t / 64, t / 64 + 4, ...
      // (16-byte coherent loads, all issued before any is used), then the 4 partial sums meet in LDS
      const auto hr = buf_rsrc(&ws->hist[0][0][0], (uint32_t)sizeof(ws->hist));
      uint4 hv[SP_C / 4];
#pragma unroll
      for (int i = 0; i < SP_C / 4; ++i) {
        const int cc = (tid >> 6) + 4 * i;
        hv[i] = buf_ld128_coh(hr, cc < C ? (uint32_t)(((cc * 2 + pass) * 256 + 4 * (tid & 63)) * 4) : 0xFFFFFFF0u);
      }
      uint4 acc = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int i = 0; i < SP_C / 4; ++i) {
        acc.x += hv[i].x;
        acc.y += hv[i].y;
        acc.z += hv[i].z;
        acc.w += hv[i].w;
      }
      __syncthreads();
      hist[tid] = 0;
      __syncthreads();
      atomicAdd(&hist[4 * (tid & 63)], (int)acc.x);
      atomicAdd(&hist[4 * (tid & 63) + 1], (int)acc.y);
      atomicAdd(&hist[4 * (tid & 63) + 2], (int)acc.z);
      atomicAdd(&hist[4 * (tid & 63) + 3], (int)acc.w);
      __syncthreads();
      int above = 0;
      const int bin = select_bin(hist, k, &above, sel);
      k -= above;
      pivot = pass == 0 ? ((uint32_t)bin << 8) : (pivot | (uint32_t)bin);
      __syncthreads();
    }
  } else {
    row_sync(ws, (unsigned)C * ++nsync, &timed_out);
  }
  // the row's max (kept entries include it), then the partial sum of exp(x - max) over kept x
  // chunk cc's value is loaded by thread cc (one round trip), then reduced over the workgroup
  float gmx = tid < C ? __uint_as_float(ld_ws(reinterpret_cast<unsigned*>(&ws->mx[tid]))) : -INFINITY;
  gmx = wg_max(gmx, red);
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < SP_PT; ++e) {
    if (bf_key(x[e]) < pivot) x[e] = -INFINITY;
    x[e] = x[e] == -INFINITY ? 0.0f : expf(x[e] - gmx);  // from here x holds exp(x - max)
    s += x[e];
  }
  s = wg_sum(s, red);
  if (tid == 0) st_ws(reinterpret_cast<unsigned*>(&ws->ps[c]), __float_as_uint(s));
  row_sync(ws, (unsigned)C * ++nsync, &timed_out);
  s = tid < C ? __uint_as_float(ld_ws(reinterpret_cast<unsigned*>(&ws->ps[tid]))) : 0.0f;
  s = wg_sum(s, red);  // a fixed reduction tree: the same sum in every chunk
  // p = bf16(exp(x - max) / sum); argmax(bf16(p / q)), the first index among equal ratios
  unsigned long long best = 0ull;
#pragma unroll
  for (int e = 0; e < SP_PT; ++e) {
    const int j = j0 + tid + e * SP_NT;
    if (j < j1) {
      const float p = rbf(x[e] / s);
      if (probs_out) probs_out[(size_t)row * V + j] = p;
      if (p != 0.0f) {  // ratio 0 never beats the kept maximum's (p > 0): no noise needed
        float q;
        if (noise) {
          q = rbf(noise[(size_t)row * V + j]);
        } else {
          const uint32_t r = philox_x0((uint32_t)j, (uint32_t)(row0 + row), off_lo, off_hi, seed_lo, seed_hi);
          const double u = ((double)(r >> 8) + 0.5) * (1.0 / 16777216.0);
          q = rbf((float)(-log(u)));
        }
        const float ratio = rbf(p / q);
        const unsigned long long key =
            ((unsigned long long)__float_as_uint(ratio) << 32) | (0xFFFFFFFFu - (uint32_t)j);
        best = key > best ? key : best;
      }
    }
  }
  best = wg_umax(best, ured);
  if (tid == 0) {
    if (best) __hip_atomic_fetch_max(&ws->best, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (timed_out) __hip_atomic_store(&ws->fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned prev = __hip_atomic_fetch_add(&ws->arrived, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == (unsigned)(C - 1);
  }
  __syncthreads();
  // every chunk's atomicMax and failure mark precede its arrival, and every chunk has left its
  // last barrier: the last one reads the row out and resets the scratch for the next call
  if (last && tid == 0) {
    const unsigned long long b =
        __hip_atomic_exchange(&ws->best, 0ull, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
    const bool failed = __hip_atomic_exchange(&ws->fail, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    tokens_out[row] = failed ? -1 : (int32_t)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull));
    __hip_atomic_store(&ws->bar, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&ws->arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

namespace {

// Rows per launch, and rows of each scratch block: 16 rows of up to SP_C chunks.
constexpr int SAMPLE_ROWS = 16;

// Scratch of fl_sample_noalloc: a fixed block per device for SAMPLE_ROWS rows (2.1 MB), part of
// the code object, so no call allocates. Host code must not pass `scratch` itself to a kernel (it
// names a host-side stand-in): its device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) SampleWs scratch[SAMPLE_ROWS];

std::mutex g_scratch_mu;
SampleWs* g_scratch_ptr[64] = {};

// Workgroups of k_sample the device holds at once (occupancy x CUs), per device, looked up on the
// first call: a launch's grid must fit, since its row barriers wait for every chunk of a row.
std::mutex g_fit_mu;
int g_fit[64] = {};
int sample_capacity(int dev) {
  std::lock_guard<std::mutex> lk(g_fit_mu);
  if (!g_fit[dev]) {
    int cu = 0, occ = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(k_sample), SP_NT, 0) !=
            hipSuccess)
      return 0;
    g_fit[dev] = cu * occ;
  }
  return g_fit[dev];
}
bool sample_coop() {
  const char* e = getenv("FLINT_AMD_COOPERATIVE");
  return e && atoi(e) != 0;
}

int sample_launch(const float* logits, int32_t rows, int32_t vocab, float temperature, int32_t top_k,
                  uint64_t seed, uint64_t offset, const float* noise, int32_t* tokens_out,
                  float* probs_out, SampleWs* wsp, void* stream) {
  const float tdiv = temperature > 1e-5f ? temperature : 1e-5f;
  const int C = std::min(SP_C, std::max(1, (vocab + SP_NT - 1) / SP_NT));  // chunks of <= SP_PT * SP_NT
  if ((vocab + C - 1) / C > SP_PT * SP_NT) return FL_E_ARG;
  int v = vocab, ci = C, tk = top_k;
  uint32_t slo = (uint32_t)seed, shi = (uint32_t)(seed >> 32), olo = (uint32_t)offset, ohi = (uint32_t)(offset >> 32);
  float td = tdiv;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return FL_E_HIP;
  const int cap = sample_capacity(dev);
  const bool coop = sample_coop();
  for (int r0 = 0; r0 < rows; r0 += SAMPLE_ROWS) {  // SAMPLE_ROWS rows per launch (the scratch's rows)
    const int n = std::min(SAMPLE_ROWS, rows - r0);
    const float* lg = logits + (size_t)r0 * vocab;
    const float* nz = noise ? noise + (size_t)r0 * vocab : nullptr;
    int32_t* to = tokens_out + r0;
    float* po = probs_out ? probs_out + (size_t)r0 * vocab : nullptr;
    int rb = r0;
    void* args[] = {(void*)&lg, &v, &ci, &rb, &td, &tk, &slo, &shi, &olo, &ohi, (void*)&nz, &to, &po, &wsp};
    if (n * C > cap) return FL_E_LAUNCH;  // the row barriers need every chunk resident at once
    // a plain launch (FLINT_AMD_COOPERATIVE=1: a cooperative one, which also guarantees residency)
    const hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
    const hipError_t e =
        coop ? hipLaunchCooperativeKernel(reinterpret_cast<const void*>(k_sample), dim3(n * C), dim3(SP_NT), args, 0, hs)
             : hipLaunchKernel(reinterpret_cast<const void*>(k_sample), dim3(n * C), dim3(SP_NT), args, 0, hs);
    if (e != hipSuccess) return FL_E_LAUNCH;
  }
  return FL_OK;
}

bool sample_args_ok(const float* logits, int32_t rows, int32_t vocab, float temperature, int32_t top_k,
                    int32_t* tokens_out) {
  return logits && tokens_out && rows >= 1 && vocab >= 1 && vocab <= SAMPLE_MAXV && top_k >= 0 &&
         temperature == temperature;  // not NaN
}

}  // namespace

extern "C" {

int fl_sample(const float* logits, int32_t rows, int32_t vocab, float temperature, int32_t top_k,
              uint64_t seed, uint64_t offset, const float* noise, int32_t* tokens_out,
              float* probs_out, void* stream) {
  if (!sample_args_ok(logits, rows, vocab, temperature, top_k, tokens_out)) return FL_E_ARG;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return FL_E_HIP;
  // per-device scratch, allocated on the first call on that device and kept until the process
  // ends; calls on one device must be stream-ordered
  static SampleWs* ws[64] = {};
  if (!ws[dev]) {
    SampleWs* w = nullptr;
    if (hipMalloc(&w, sizeof(SampleWs) * SAMPLE_ROWS) != hipSuccess) return FL_E_HIP;
    if (hipMemset(w, 0, sizeof(SampleWs) * SAMPLE_ROWS) != hipSuccess) return FL_E_HIP;
    ws[dev] = w;
  }
  return sample_launch(logits, rows, vocab, temperature, top_k, seed, offset, noise, tokens_out,
                       probs_out, ws[dev], stream);
}

int fl_sample_noalloc(const float* logits, int32_t rows, int32_t vocab, float temperature,
                      int32_t top_k, uint64_t seed, uint64_t offset, const float* noise,
                      int32_t* tokens_out, float* probs_out, void* stream) {
  if (!sample_args_ok(logits, rows, vocab, temperature, top_k, tokens_out)) return FL_E_ARG;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return FL_E_HIP;
  SampleWs* wsp;
  {
    // the device address of this device's copy of `scratch`, looked up once (with the device
    // current: each device holds its own copy at its own address)
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
      void* p = nullptr;
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return FL_E_HIP;
      g_scratch_ptr[dev] = reinterpret_cast<SampleWs*>(p);
    }
    wsp = g_scratch_ptr[dev];
  }
  return sample_launch(logits, rows, vocab, temperature, top_k, seed, offset, noise, tokens_out,
                       probs_out, wsp, stream);
}

}  // extern "C"
