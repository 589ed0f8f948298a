// Temperature / top-k sampling of logit rows on the GPU (reference engine/generate.py:36-55).
//
// One workgroup per row keeps the row in LDS as bf16 (up to 65536 values, 128 KB) and applies
// the reference's steps with its bf16 rounding points: x = bf16(l / max(T, 1e-5)); the
// top-k pivot is the k-th largest x, found by a two-pass radix select over the 16-bit ordered
// keys of the bf16 values (256-bin LDS histograms); x < pivot drops out; p = bf16(exp(x - max)
// / sum); q = bf16(-log(u)) with u from Philox4x32-10 keyed by the caller's seed, or q given;
// the sample is the first index of the largest bf16(p / q), which is
// multinomial_sample_one_no_sync's argmax(probs / exponential noise).
#include "fl_common.h"

namespace {

constexpr int SAMPLE_NT = 1024;
constexpr int SAMPLE_MAXV = 65536;            // vocab limit: the row lives in LDS as bf16
constexpr int SAMPLE_NWAVE = SAMPLE_NT / FL_WAVE;

// Philox4x32-10 (Salmon et al., SC 2011): 10 rounds of two 32x32->64 multiplies, Weyl key bumps
__device__ __forceinline__ uint32_t philox_x0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                              uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c0 = n0;
    c1 = (uint32_t)p1;
    c2 = n2;
    c3 = (uint32_t)p0;
  }
  return c0;
}

// ordered 16-bit key of a bf16 value: larger value <-> larger key
__device__ __forceinline__ uint32_t bf_key(float x) {
  const uint32_t b = __float_as_uint(x) >> 16;
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

__device__ __forceinline__ float block_max(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = red[0];
  for (int w = 1; w < SAMPLE_NWAVE; ++w) v = fmaxf(v, red[w]);
  return v;
}
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = 0.0f;
  for (int w = 0; w < SAMPLE_NWAVE; ++w) v += red[w];
  return v;
}
__device__ __forceinline__ unsigned long long block_umax(unsigned long long v, unsigned long long* red) {
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
  for (int w = 1; w < SAMPLE_NWAVE; ++w) v = red[w] > v ? red[w] : v;
  return v;
}

// The bin of a 256-bin histogram (counts in hist) that holds the k-th largest key, scanning from
// bin 255 down: returns the bin and, through above, how many keys lie in higher bins. Wave 0
// scans (lane l owns bins 4l..4l+3); the result goes to every thread through sel.
__device__ __forceinline__ int select_bin(const int* hist, int k, int* above, int* sel) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    const int b0 = 4 * tid;
    const int c0 = hist[b0], c1 = hist[b0 + 1], c2 = hist[b0 + 2], c3 = hist[b0 + 3];
    const int own = c0 + c1 + c2 + c3;
    int incl = own;  // sum over lanes >= tid
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_down(incl, o, 64);
      if (tid + o < 64) incl += t;
    }
    const int hi = incl - own;  // keys in bins above this lane's four
    if (hi < k && incl >= k) {
      // the highest of the four bins where the running count from the top reaches k
      int bin, acc;
      if (hi + c3 >= k) {
        bin = b0 + 3, acc = hi;
      } else if (hi + c3 + c2 >= k) {
        bin = b0 + 2, acc = hi + c3;
      } else if (hi + c3 + c2 + c1 >= k) {
        bin = b0 + 1, acc = hi + c3 + c2;
      } else {
        bin = b0, acc = hi + c3 + c2 + c1;
      }
      sel[0] = bin;
      sel[1] = acc;
    }
  }
  __syncthreads();
  const int bin = sel[0];
  *above = sel[1];
  return bin;
}

// LDS: the row as bf16 (vocab values, padded to 16 bytes), then the per-wave histograms
inline size_t sample_lds_bytes(int V) { return (((size_t)V * 2 + 15) & ~(size_t)15) + SAMPLE_NWAVE * 256 * 4; }

__global__ __launch_bounds__(SAMPLE_NT) void k_sample(const float* __restrict__ logits, int V,
                                                      float tdiv, int top_k, uint32_t seed_lo,
                                                      uint32_t seed_hi, uint32_t off_lo,
                                                      uint32_t off_hi, const float* __restrict__ noise,
                                                      int32_t* __restrict__ tokens_out,
                                                      float* __restrict__ probs_out) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  int* whist = reinterpret_cast<int*>(smem + (((size_t)V * 2 + 15) & ~(size_t)15));
  __shared__ int hist[256];
  __shared__ int sel[2];
  __shared__ float red[SAMPLE_NWAVE];
  __shared__ unsigned long long ured[SAMPLE_NWAVE];
  const int tid = threadIdx.x, row = blockIdx.x;
  const float* lg = logits + (size_t)row * V;
  // x = bf16(bf16(logit) / max(T, 1e-5))  (generate.py:42)
  for (int j = tid; j < V; j += SAMPLE_NT) xs[j] = (uint16_t)f2bf(rbf(lg[j]) / tdiv);
  __syncthreads();
  // top-k pivot (generate.py:44-47): keys >= the k-th largest key stay. Each wave counts into
  // its own histogram (the keys of a row crowd into a few bins), the 16 are summed, and the bin
  // holding the k-th largest key is selected: first over the high byte, then over the low byte
  // of the keys in that bin.
  uint32_t pivot = 0;
  if (top_k > 0 && top_k < V) {
    int k = top_k;
    auto count = [&](bool low) {
      for (int b = tid; b < SAMPLE_NWAVE * 256; b += SAMPLE_NT) whist[b] = 0;
      __syncthreads();
      int* h = whist + (tid >> 6) * 256;
      for (int j = tid; j < V; j += SAMPLE_NT) {
        const uint32_t key = bf_key(bf2f(xs[j]));
        if (!low || (key >> 8) == (pivot >> 8)) atomicAdd(&h[low ? (key & 0xFFu) : (key >> 8)], 1);
      }
      __syncthreads();
      if (tid < 256) {
        int c = 0;
        for (int w = 0; w < SAMPLE_NWAVE; ++w) c += whist[w * 256 + tid];
        hist[tid] = c;
      }
      __syncthreads();
      int above = 0;
      const int bin = select_bin(hist, k, &above, sel);
      k -= above;
      __syncthreads();
      return bin;
    };
    pivot = (uint32_t)count(false) << 8;
    pivot |= (uint32_t)count(true);
  }
  float mx = -INFINITY;
  for (int j = tid; j < V; j += SAMPLE_NT) {  // drop x < pivot (bf16 -inf is 0xFF80)
    float x = bf2f(xs[j]);
    if (bf_key(x) < pivot) {
      xs[j] = 0xFF80u;
      x = -INFINITY;
    }
    mx = fmaxf(mx, x);
  }
  mx = block_max(mx, red);
  // softmax (generate.py:48): p = bf16(exp(x - max) / sum); exp is evaluated again below
  auto ex = [&](int j) {
    const float v = bf2f(xs[j]);
    return v == -INFINITY ? 0.0f : expf(v - mx);
  };
  float s = 0.0f;
  for (int j = tid; j < V; j += SAMPLE_NT) s += ex(j);
  s = block_sum(s, red);
  // argmax(bf16(p / q)), the first index among equal ratios (generate.py:36-38)
  unsigned long long best = 0ull;
  for (int j = tid; j < V; j += SAMPLE_NT) {
    const float p = rbf(ex(j) / s);
    if (probs_out) probs_out[(size_t)row * V + j] = p;
    if (p == 0.0f) continue;  // ratio 0 never beats the kept maximum's (p > 0): no noise needed
    float q;
    if (noise) {
      q = rbf(noise[(size_t)row * V + j]);
    } else {
      const uint32_t r = philox_x0((uint32_t)j, (uint32_t)row, off_lo, off_hi, seed_lo, seed_hi);
      const double u = ((double)(r >> 8) + 0.5) * (1.0 / 16777216.0);
      q = rbf((float)(-log(u)));
    }
    const float ratio = rbf(p / q);
    const unsigned long long key =
        ((unsigned long long)__float_as_uint(ratio) << 32) | (0xFFFFFFFFu - (uint32_t)j);
    best = key > best ? key : best;
  }
  best = block_umax(best, ured);
  if (tid == 0) tokens_out[row] = (int32_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
}

}  // namespace

extern "C" {

int fl_sample(const float* logits, int32_t rows, int32_t vocab, float temperature, int32_t top_k,
              uint64_t seed, uint64_t offset, const float* noise, int32_t* tokens_out,
              float* probs_out, void* stream) {
  if (!logits || !tokens_out || rows < 1 || vocab < 1 || vocab > SAMPLE_MAXV || top_k < 0)
    return FL_E_ARG;
  if (!(temperature == temperature)) return FL_E_ARG;  // NaN
  const float tdiv = temperature > 1e-5f ? temperature : 1e-5f;
  const size_t lds = sample_lds_bytes(vocab);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FL_E_HIP;
  static unsigned long long lds_set = 0;  // devices whose LDS limit for k_sample is raised
  if (dev < 64 && !(lds_set & (1ull << dev))) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(k_sample), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)sample_lds_bytes(SAMPLE_MAXV)) != hipSuccess)
      return FL_E_HIP;
    lds_set |= 1ull << dev;
  }
  hipLaunchKernelGGL(k_sample, dim3(rows), dim3(SAMPLE_NT), lds, reinterpret_cast<hipStream_t>(stream),
                     logits, vocab, tdiv, top_k, (uint32_t)seed, (uint32_t)(seed >> 32), (uint32_t)offset,
                     (uint32_t)(offset >> 32), noise, tokens_out, probs_out);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

}  // extern "C"
