// int4 group quantisation, bit-exact dequantisation and the standalone M=1 int4 GEMV.
//
// Quantisation restates gpt-fast's asymmetric group scheme (reference engine/quantize.py:58-76,
// :102-128, :131-135): every step is a bf16 tensor op in the reference, so every step here
// computes in fp32 and rounds to bf16 (RNE) at the same points.
#include "fl_common.h"
#include <algorithm>

namespace {

constexpr uint32_t kBf16OneEMinus6 = 0x3586u;  // bf16(1e-6): clamp(min=1e-6) on a bf16 tensor

// One thread per packed word (8 elements); 16 consecutive threads form one (row, 128-group).
__global__ __launch_bounds__(256) void k_quantize(const uint16_t* __restrict__ w,
                                                  uint32_t* __restrict__ q,
                                                  uint32_t* __restrict__ sz, int64_t nwords) {
  const int64_t word = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = word < nwords;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (valid) v = *reinterpret_cast<const uint4*>(w + word * 8);
  const uint32_t pk[4] = {v.x, v.y, v.z, v.w};
  float x[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[2 * j] = bflo(pk[j]);
    x[2 * j + 1] = bfhi(pk[j]);
  }
  float mx = x[0], mn = x[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) {
    mx = fmaxf(mx, x[e]);
    mn = fminf(mn, x[e]);
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    mn = fminf(mn, __shfl_xor(mn, o, 64));
  }
  // get_group_qparams (quantize.py:71-74)
  float d = rbf(mx - mn);
  d = fmaxf(d, bf2f(kBf16OneEMinus6));
  const float scale = rbf(d / 15.0f);
  const float s8 = rbf(scale * 8.0f);
  const float zero = rbf(mn + s8);
  // group_quantize_tensor_from_qparams (quantize.py:116-126)
  const float minv = rbf(zero - s8);
  uint32_t word_q = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float t = rbf(x[e] - minv);
    t = rbf(t / scale);
    float r = rbf(rintf(t));
    r = fminf(fmaxf(r, 0.0f), 15.0f);
    word_q |= ((uint32_t)r) << (4 * nib_pos(e));
  }
  if (valid) {
    q[word] = word_q;
    if ((word & 15) == 0) sz[word >> 4] = f2bf(scale) | (f2bf(zero) << 16);
  }
}

// One thread per 16-byte chunk (4 packed words, 32 elements of one group): bf16 outputs through
// the same dequantisation sequence the GEMVs use -- dq32 on the vector ALUs (MX = false: the
// M <= 32 GEMM of this file) or dq32_mx on the matrix cores (MX = true: the M = 1 GEMVs of this
// file and the decode kernel's; the verify tiles run the tiled form, fl_dequant_int4_tiled's). Threads 4b..4b+3 hold the four chunks of one group (nchunks is a
// multiple of 4), as dq32_mx needs; every thread runs it (past the end on the last chunk) so
// that all lanes of a wave run the matrix-core steps together.
template <bool MX>
__global__ __launch_bounds__(256) void k_dequant(const uint32_t* __restrict__ q,
                                                 const uint32_t* __restrict__ sz,
                                                 uint16_t* __restrict__ out, int64_t nchunks) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if constexpr (!MX) {
    if (c >= nchunks) return;
  }
  const int64_t cc = c < nchunks ? c : nchunks - 1;
  uint32_t d[4][4];
  if constexpr (MX)
    dq32_mx(reinterpret_cast<const uint4*>(q)[cc], sz[cc >> 2], mx_lane(), d);
  else
    dq32(reinterpret_cast<const uint4*>(q)[cc], dq_const(sz[cc >> 2]), d);
  if (c >= nchunks) return;
  uint4* o = reinterpret_cast<uint4*>(out + c * 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = make_uint4(d[0][i], d[1][i], d[2][i], d[3][i]);
}

// M=1 GEMV. A workgroup owns `rows_per_wg` consecutive rows, whose packed words form one
// contiguous block; its 16-byte chunks (32 elements each) are dealt round-robin over the
// threads so that every thread gets the same number of chunks and every load is coalesced
// (threads 4b..4b+3 take the four chunks of one group, as the matrix-core dequantisation's lane
// blocks need). Per-chunk partial sums go to LDS and each row is summed there in a fixed order.
constexpr int kGemvThreads = 256;
constexpr int kGemvMaxChunks = 8;  // per thread

__global__ __launch_bounds__(kGemvThreads) void k_gemv(const uint32_t* __restrict__ q,
                                                       const uint32_t* __restrict__ sz,
                                                       const uint16_t* __restrict__ x,
                                                       uint16_t* __restrict__ y, int n, int k,
                                                       int rows_per_wg) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* part = reinterpret_cast<float*>(smem + (size_t)k * 2);
  const int tid = threadIdx.x;
  const int r0 = blockIdx.x * rows_per_wg;
  const int rows = min(rows_per_wg, n - r0);
  const int cpr = k >> 5;  // chunks per row
  const int total = rows * cpr;
  const uint4* wblk = reinterpret_cast<const uint4*>(q + (size_t)r0 * (k >> 3));
  const uint32_t* sblk = sz + (size_t)r0 * (k >> 7);

  // issue the weight loads first: they do not depend on x
  uint4 wr[kGemvMaxChunks];
  uint32_t sr[kGemvMaxChunks];
#pragma unroll
  for (int i = 0; i < kGemvMaxChunks; ++i) {
    const int f = tid + i * kGemvThreads;
    if (f < total) {
      wr[i] = wblk[f];
      sr[i] = sblk[f >> 2];
    }
  }
  for (int i = tid; i < (k >> 3); i += kGemvThreads)
    reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(x)[i];
  __syncthreads();
  int c = tid % cpr;
  const int step = kGemvThreads % cpr;
#pragma unroll
  for (int i = 0; i < kGemvMaxChunks; ++i) {
    const int f = tid + i * kGemvThreads;
    if (f < total) {
      const uint4* x4 = reinterpret_cast<const uint4*>(xs + c * 32);
      part[f] = chunk_dot_mx(wr[i], sr[i], x4, 0.0f);
    }
    c += step;
    if (c >= cpr) c -= cpr;
  }
  __syncthreads();
  // row reduction: L lanes per row, L = largest power of two <= threads/rows (<= 64)
  int L = 64;
  while (L * rows > kGemvThreads) L >>= 1;
  const int row = tid / L, li = tid % L;
  float acc = 0.0f;
  if (row < rows)
    for (int j = li; j < cpr; j += L) acc += part[row * cpr + j];
  acc = group_sum(acc, L);
  if (row < rows && li == 0) y[r0 + row] = (uint16_t)f2bf(acc);
}

// M=1 GEMV streamed by persistent waves (the shapes whose K is 2560 or 8192, i.e. every int4
// layer of the 3B model). GV_WG workgroups of GV_NW waves per CU, four waves per SIMD (at most
// 128 VGPRs: one chunk's dequantisation temporaries live at a time); a wave takes tiles of 64 >> LG
// rows, 2^LG lanes per row and C 16-byte chunks per lane (one row's K / 32 chunks exactly), and
// walks tiles t, t + W, t + 2W, ... (W waves in the grid) with two register buffers: the next
// tile's weights are requested before the current tile is dequantised, so the HBM stream and
// the VALU work overlap instead of every workgroup loading, then computing. The activation
// vector is staged in LDS once per workgroup (its requests go out first, ahead of the weights,
// so the first tile does not wait behind them). A row's partial sums meet in a DPP reduction
// over its lanes (fixed order); its first lane writes y. All loads are range-checked buffer
// loads (tiles past N read zeros and store nothing), so no load sits under a branch. With 16 or
// 64 lanes per row, lanes 4b..4b+3 always hold the four chunks of one group (dq32_mx's blocks).
constexpr int GV_NW = 8;
constexpr int GV_NT = GV_NW * 64;
constexpr int GV_WG = 2;  // workgroups per CU (four waves per SIMD hide more of the HBM latency than
                          // two: steady-state streaming +7% at K = 2560, +15% at K = 8192)

template <int LG, int C>
__device__ __forceinline__ void gv_load(__amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t sr, int t, int n,
                                        int cpr, int gpr, uint4 (&w)[C], uint32_t (&s)[C]) {
  const int lane = threadIdx.x & 63;
  const int row = t * (64 >> LG) + (lane >> LG), j = lane & ((1 << LG) - 1);
  const bool ok = row < n;
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = j + (i << LG);
    w[i] = buf_ld128(wr, ok ? (uint32_t)(row * cpr + c) * 16u : 0xFFFFFFF0u);
    s[i] = buf_ld32(sr, ok ? (uint32_t)(row * gpr + (c >> 2)) * 4u : 0xFFFFFFF0u);
  }
}

template <int LG, int C>
__device__ __forceinline__ void gv_tile(const uint4* xs, int t, int n, const uint4 (&w)[C],
                                        const uint32_t (&s)[C], uint16_t* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int row = t * (64 >> LG) + (lane >> LG), j = lane & ((1 << LG) - 1);
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = j + (i << LG);
    acc = chunk_dot_mx(w[i], s[i], xs + 5 * c, acc);  // chunk c's 4 x slots start at 5c (bank spread)
    __builtin_amdgcn_sched_barrier(0);              // one chunk's temporaries live at a time
  }
  acc = group_sum(acc, 1 << LG);
  if (j == 0 && row < n) y[row] = (uint16_t)f2bf(acc);
}

template <int LG, int C>
__global__ __launch_bounds__(GV_NT, 4) void k_gemv_stream(const uint32_t* __restrict__ q,
                                                          const uint32_t* __restrict__ sz,
                                                          const uint16_t* __restrict__ x,
                                                          uint16_t* __restrict__ y, int n, int k) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint4* xs = reinterpret_cast<uint4*>(smem);  // x: logical slot v at v + v / 4
  const int tid = threadIdx.x, wave = tid >> 6;
  const int cpr = k >> 5, gpr = k >> 7;
  const int ntiles = (n + (64 >> LG) - 1) / (64 >> LG);
  const int W = gridDim.x * GV_NW;
  const auto xr = buf_rsrc(x, (uint32_t)k * 2u);
  const auto wr = buf_rsrc(q, (uint32_t)n * (uint32_t)(k >> 1));
  const auto sr = buf_rsrc(sz, (uint32_t)n * (uint32_t)gpr * 4u);
  constexpr int XPT = 8192 / 8 / GV_NT;  // 16-byte x slots per thread (k <= 8192)
  uint4 xv[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) xv[i] = buf_ld128(xr, (uint32_t)(tid + i * GV_NT) * 16u);
  uint4 wa[C], wb[C];
  uint32_t sa[C], sb[C];
  int t = blockIdx.x * GV_NW + wave;
  // a wave takes tiles in pairs (t, t + W): both tiles' requests go out together, then both are
  // computed (no register buffer is carried across the loop, so nothing has to be copied)
  gv_load<LG, C>(wr, sr, t, n, cpr, gpr, wa, sa);
  gv_load<LG, C>(wr, sr, t + W, n, cpr, gpr, wb, sb);
  __builtin_amdgcn_sched_barrier(0);
  // every thread stores its slots (the LDS holds XPT * GV_NT of them; slots past K hold zeros),
  // so no store, and no load feeding one, sits under a branch that would wait for every load
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int v = tid + i * GV_NT;
    xs[v + (v >> 2)] = xv[i];
  }
  lds_barrier();
  while (t < ntiles) {
    gv_tile<LG, C>(xs, t, n, wa, sa, y);
    if (t + W < ntiles) gv_tile<LG, C>(xs, t + W, n, wb, sb, y);
    t += 2 * W;
    if (t >= ntiles) break;
    gv_load<LG, C>(wr, sr, t, n, cpr, gpr, wa, sa);
    gv_load<LG, C>(wr, sr, t + W, n, cpr, gpr, wb, sb);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Y[M, N] = bf16(X[M, K] . dq[N, K]^T), 1 <= M <= 16, on the matrix cores: one workgroup of 4
// waves per 16-row tile of W; the waves take the K/128 groups round-robin, each lane dequantises
// one 16-byte chunk per group (row n0 + l%16, chunk l/16) and feeds it to four MFMA steps, so
// every weight is read and dequantised once for all M rows. Activation fragments are read from
// global memory (rows >= M and rows >= N come back as zero from range-checked loads); the four
// waves' partial tiles are summed in LDS in a fixed order.
constexpr int kGemmWaves = 4;

__global__ __launch_bounds__(64 * kGemmWaves) void k_gemm(const uint32_t* __restrict__ q,
                                                          const uint32_t* __restrict__ sz,
                                                          const uint16_t* __restrict__ x,
                                                          uint16_t* __restrict__ y, int m, int n,
                                                          int k) {
  __shared__ float part[kGemmWaves][2][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, c = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int rows = min(16, n - n0);
  const int groups = k >> 7;
  const bool two = m > 16;  // a second 16-row block of activations (tokens 16..31)
  const auto wr = buf_rsrc(q + (size_t)n0 * (k >> 3), (uint32_t)rows * (uint32_t)(k >> 1));
  const auto sr = buf_rsrc(sz + (size_t)n0 * groups, (uint32_t)rows * (uint32_t)groups * 4u);
  const auto xr = buf_rsrc(x, (uint32_t)m * (uint32_t)k * 2u);
  const uint32_t woff = (uint32_t)r * (uint32_t)(k >> 1) + (uint32_t)c * 16u;   // bytes
  const uint32_t xoff = (uint32_t)r * (uint32_t)k * 2u + (uint32_t)c * 64u;     // bytes
  const uint32_t xoff2 = xoff + 16u * (uint32_t)k * 2u;
  fl_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int u = wave; u < groups; u += kGemmWaves) {
    const uint4 w = buf_ld128(wr, woff + (uint32_t)u * 64u);
    const uint32_t s = buf_ld32(sr, ((uint32_t)r * (uint32_t)groups + (uint32_t)u) * 4u);
    uint4 xa[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) xa[e] = buf_ld128(xr, xoff + (uint32_t)u * 256u + (uint32_t)e * 16u);
    uint32_t d[4][4];
    dq32(w, dq_const(s), d);
    mfma_chunk(d, xa, acc);
    if (two) {
#pragma unroll
      for (int e = 0; e < 4; ++e) xa[e] = buf_ld128(xr, xoff2 + (uint32_t)u * 256u + (uint32_t)e * 16u);
      mfma_chunk(d, xa, acc2);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    part[wave][0][(c * 4 + i) * 16 + r] = acc[i];
    part[wave][1][(c * 4 + i) * 16 + r] = acc2[i];
  }
  __syncthreads();
  for (int t = threadIdx.x; t < (two ? 512 : 256); t += 64 * kGemmWaves) {
    const int row = t >> 4, col = t & 15;  // activation row (token), weight row in the tile
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kGemmWaves; ++w) v += part[w][t >> 8][t & 255];
    if (row < m && col < rows) y[(size_t)row * n + n0 + col] = (uint16_t)f2bf(v);
  }
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

int fl_version(void) { return 1; }

int fl_quantize_int4(const uint16_t* w, uint32_t* q, uint32_t* sz, int32_t n, int32_t k,
                     void* stream) {
  if (!w || !q || !sz || n <= 0 || k <= 0 || (k % FL_GROUP) != 0) return FL_E_ARG;
  const int64_t nwords = (int64_t)n * (k / 8);
  const int64_t blocks = (nwords + 255) / 256;
  if (blocks > 0x7FFFFFFF) return FL_E_ARG;
  hipLaunchKernelGGL(k_quantize, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), w, q, sz,
                     nwords);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

int fl_dequant_int4(const uint32_t* q, const uint32_t* sz, uint16_t* out, int32_t n, int32_t k,
                    void* stream) {
  if (!q || !sz || !out || n <= 0 || k <= 0 || (k % FL_GROUP) != 0) return FL_E_ARG;
  const int64_t nchunks = (int64_t)n * (k / 32);
  const int64_t blocks = (nchunks + 255) / 256;
  if (blocks > 0x7FFFFFFF) return FL_E_ARG;
  hipLaunchKernelGGL(k_dequant<false>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), q, sz,
                     out, nchunks);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

int fl_dequant_int4_mx(const uint32_t* q, const uint32_t* sz, uint16_t* out, int32_t n, int32_t k,
                       void* stream) {
  if (!q || !sz || !out || n <= 0 || k <= 0 || (k % FL_GROUP) != 0) return FL_E_ARG;
  const int64_t nchunks = (int64_t)n * (k / 32);
  const int64_t blocks = (nchunks + 255) / 256;
  if (blocks > 0x7FFFFFFF) return FL_E_ARG;
  hipLaunchKernelGGL(k_dequant<true>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), q, sz,
                     out, nchunks);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

int fl_gemv_int4(const uint32_t* q, const uint32_t* sz, const uint16_t* x, uint16_t* y, int32_t n,
                 int32_t k, void* stream) {
  if (!q || !sz || !x || !y || n <= 0 || k <= 0 || (k % FL_GROUP) != 0 || k > 16384)
    return FL_E_ARG;
  // K = 2560 / 8192: the streamed kernel, GV_WG workgroups per CU (fewer when N has fewer tiles)
  if ((k == 2560 || k == 8192) && (int64_t)n * (k / 2) <= 0x7FFFFFFFll) {
    const void* kern = k == 2560 ? reinterpret_cast<const void*>(k_gemv_stream<4, 5>)
                                 : reinterpret_cast<const void*>(k_gemv_stream<6, 4>);
    const int rpt = k == 2560 ? 4 : 1;
    static int cus = 0;
    if (!cus) {
      int dev = 0;
      if (hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        return FL_E_HIP;
    }
    const int tiles = (n + rpt - 1) / rpt;
    const int blocks = std::min(GV_WG * cus, (tiles + GV_NW - 1) / GV_NW);
    const size_t shm = (size_t)(8192 / 8 + 8192 / 32) * 16;  // every thread's x slots (k <= 8192)
    const int nn = n, kk = k;
    void* args[] = {(void*)&q, (void*)&sz, (void*)&x, (void*)&y, (void*)&nn, (void*)&kk};
    return hipLaunchKernel(kern, dim3(blocks), dim3(GV_NT), args, shm, as_stream(stream)) == hipSuccess
               ? FL_OK : FL_E_LAUNCH;
  }
  const int cpr = k / 32;
  // rows per workgroup: as many as keep every thread at <= kGemvMaxChunks chunks, at most 16
  int rows = (kGemvThreads * kGemvMaxChunks) / cpr;
  if (rows > 8) rows = 8;
  if (rows < 1) return FL_E_ARG;
  const int blocks = (n + rows - 1) / rows;
  const size_t shm = (size_t)k * 2 + (size_t)rows * cpr * 4;
  hipLaunchKernelGGL(k_gemv, dim3(blocks), dim3(kGemvThreads), shm, as_stream(stream), q, sz, x, y,
                     n, k, rows);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

int fl_gemm_int4(const uint32_t* q, const uint32_t* sz, const uint16_t* x, uint16_t* y, int32_t m,
                 int32_t n, int32_t k, void* stream) {
  if (!q || !sz || !x || !y || n <= 0 || k <= 0 || (k % FL_GROUP) != 0) return FL_E_ARG;
  if (m < 1 || m > FL_MAX_VERIFY) return FL_E_M;
  if ((int64_t)n * (k / 2) > 0xFFFFFFFFll || (int64_t)m * k * 2 > 0xFFFFFFFFll) return FL_E_ARG;
  hipLaunchKernelGGL(k_gemm, dim3((n + 15) / 16), dim3(64 * kGemmWaves), 0, as_stream(stream), q,
                     sz, x, y, m, n, k);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

}  // extern "C"
