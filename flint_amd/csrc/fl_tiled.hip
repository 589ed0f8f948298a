// int4 GEMV whose exact dequantisation runs on the matrix cores, over a tiled weight layout.
//
// The dequantisation contract is the same as everywhere in this library, gpt-fast's
// bf16(bf16((q - 8) * s) + z) (reference engine/quantize.py:138-155), and y = bf16(sum x * dq) with
// fp32 accumulation (quantize.py:517-525). Here the two exact fp32 steps and the dot run as MFMAs:
//   D1 = A1 . diag(s) + C1:  A1 = (128 + q) as bf16 (one AND-OR per two weights puts the nibble in
//        the mantissa of 128.0), C1 = -136 s, so D1 = (q - 8) s exactly (one nonzero product);
//        v_cvt_pk_bf16_f32 rounds it to bf16 (RNE), the reference's first rounding;
//   D2 = I . a + C2:  C2 = z, so D2 = fp32(a + z), the reference's fp32 add; cvt rounds it again;
//   D3 += x . dq  (16x16x32 MFMA over two 16-position tiles; for M = 1 every output row holds the
//        same sum, for M <= 16 token rows one row each).
// Both dequantisation steps are v_mfma_f32_4x4x4_16b_bf16: 16 independent 4x4x4 products, block
// b on lanes 4b..4b+3 (row i of A from lane 4b + i, column j of B from lane 4b + j, column j of D
// to lane 4b + j). With A1 = four rows at one column per lane and B1 = diag(s) (lane 4b + j puts
// the scale of its own row in slot j), lane 4b + j receives, in slot i, lane 4b + i's value of row
// j times row j's scale: the block transposes, so every lane ends with four columns of one row.
// Both have one nonzero product per output plus the accumulator, so their fp32 results are
// exactly the reference's (D1 is exactly representable; D2 is one fp32 addition, and where that
// addition rounds, |a| is below 2^-16 |z| and the bf16 rounding gives z either way).
//
// Tiled layout (fl_tile_int4 converts this library's row layout into it): for each block of 16 rows
// and each 128-column group, 1 KB; lane L of a wave reads the 16 bytes at L * 16: rows
// 4 p .. 4 p + 3 with p = (L / 4) % 4, at the 8 columns c + 16 t (t = 0..7), c = 4 (L / 16) + L % 4:
//   word 0: bits 4t..4t+3 = q[4p][c + 16t], bits 16+4t.. = q[4p+1][c + 16t]   (t = 0..3)
//   word 1: the same for t = 4..7;  words 2 / 3: rows 4p+2 / 4p+3.
// After D1 and D2, lane L holds row L % 16 at columns 4 (L / 16) .. + 3 of each tile: the B
// fragment of the 16x16x32 dot for two tiles. Scale / zero words stay [N, K/128]. The unit
// routines (unit_dq_t, unit_mma_t) live in fl_common.h: the verify kernel runs them too.
#include "fl_common.h"
#include <algorithm>

namespace {

// row layout -> tiled layout: one thread per 16-byte tiled chunk
__global__ __launch_bounds__(256) void k_tile_int4(const uint32_t* __restrict__ q, uint4* __restrict__ qt,
                                                   int n, int k) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int G = k >> 7;
  const int64_t chunks = (int64_t)(n >> 4) * G * 64;
  if (idx >= chunks) return;
  const int l = (int)(idx & 63), p = (l >> 2) & 3, c = 4 * (l >> 4) + (l & 3);
  const int64_t blk = idx >> 6;
  const int g = (int)(blk % G), rb = (int)(blk / G);
  const int kw = k >> 3;  // words per row
  auto nib = [&](int r, int col) -> uint32_t {  // q[r][col] of the row layout
    const uint32_t w = q[(size_t)r * kw + (col >> 3)];
    return (w >> (4 * nib_pos(col & 7))) & 0xFu;
  };
  uint32_t wd[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int h = 0; h < 2; ++h) {      // rows 4p + 2h, 4p + 2h + 1 -> words 2h, 2h + 1
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int col = g * 128 + c + 16 * t;
      const int r = rb * 16 + 4 * p + 2 * h;
      const uint32_t v = nib(r, col) | (nib(r + 1, col) << 16);
      wd[2 * h + (t >> 2)] |= v << (4 * (t & 3));
    }
  }
  qt[idx] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
}

// One 1 KB unit (16 rows x one 128-group) of the tiled matrix, dequantised and dotted with x:
// acc += x[group] . dq^T (every output row of the MFMA holds the same sum). w: this lane's 16
// bytes; xs: x in LDS (bf16, plain order).
__device__ __forceinline__ void unit_dot(uint4 w, uint32_t szw, const uint16_t* xs, int g, const MxLane& m,
                                         fl_f32x4& acc) {
  const int b = (threadIdx.x & 63) >> 4;
  unit_mma_t<8>(w, szw, m, xs + g * 128 + 4 * b, acc);
}

// y = bf16(W x): one workgroup of TW_NW waves per 16-row block (blocks strided over the grid); the
// waves take the block's 128-groups round-robin, their partial sums meet in LDS in wave order.
constexpr int TW_NW = 4;
__global__ __launch_bounds__(TW_NW * 64) void k_gemv_tiled(const uint4* __restrict__ qt, const uint32_t* __restrict__ sz,
                                                           const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                           int n, int k) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* part = reinterpret_cast<float*>(smem + (size_t)k * 2);  // [TW_NW][16]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = k >> 7, nb = n >> 4;
  for (int i = tid; i < (k >> 3); i += TW_NW * 64)
    reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(x)[i];
  __syncthreads();
  const int c = lane & 15;
  const MxLane m = mx_lane();
  for (int rb = blockIdx.x; rb < nb; rb += gridDim.x) {
    fl_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint4* blk = qt + (size_t)rb * G * 64;
    const uint32_t* srow = sz + (size_t)(rb * 16 + c) * G;
    for (int g = wave; g < G; g += TW_NW) unit_dot(blk[(size_t)g * 64 + lane], srow[g], xs, g, m, acc);
    if (lane < 16) part[wave * 16 + lane] = acc[0];
    __syncthreads();
    if (tid < 16) {
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < TW_NW; ++w) v += part[w * 16 + tid];
      y[rb * 16 + tid] = (uint16_t)f2bf(v);
    }
    __syncthreads();
  }
}

// The same GEMV with every unit a wave computes requested up front: one workgroup of NW waves
// per 16-row block, wave w taking the block's groups w, w + NW, ... (at most UPW of them, all in
// registers). x is requested first and the weights after it (loads complete in order, so the x
// staging waits for x alone), then each unit is computed as its bytes arrive. In the loop kernel
// above a wave requests a unit only after the previous one is done, so every unit pays a full
// memory latency.
template <int NW, int UPW>
__global__ __launch_bounds__(NW * 64) void k_gemv_tiled_pf(const uint4* __restrict__ qt, const uint32_t* __restrict__ sz,
                                                           const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                           int n, int k) {
  // x slots: XPT per thread cover K <= NW * UPW * 128 (slots past K hold zeros, never read)
  constexpr int XPT = UPW * 128 / 8 / 64;
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* part = reinterpret_cast<float*>(smem + (size_t)XPT * NW * 64 * 16);  // [NW][16]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = k >> 7, nb = n >> 4, nx = k >> 3;
  const auto xr = buf_rsrc(x, (uint32_t)k * 2u);
  uint4 xv[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int v = tid + i * NW * 64;
    xv[i] = buf_ld128(xr, v < nx ? (uint32_t)v * 16u : 0xFFFFFFF0u);
  }
  const int c = lane & 15;
  const MxLane m = mx_lane();
  bool staged = false;
  for (int rb = blockIdx.x; rb < nb; rb += gridDim.x) {
    const auto wr = buf_rsrc(qt + (size_t)rb * G * 64, (uint32_t)G * 1024u);
    const auto sr = buf_rsrc(sz + (size_t)rb * 16 * G, (uint32_t)G * 64u);
    uint4 w[UPW];
    uint32_t sw[UPW];
#pragma unroll
    for (int i = 0; i < UPW; ++i) {  // units past G: no memory access
      const int g = wave + NW * i;
      w[i] = buf_ld128(wr, g < G ? (uint32_t)(g * 64 + lane) * 16u : 0xFFFFFFF0u);
      sw[i] = buf_ld32(sr, g < G ? (uint32_t)(c * G + g) * 4u : 0xFFFFFFF0u);
    }
    if (!staged) {  // every thread stores its slots (no store under a branch that waits for all loads)
#pragma unroll
      for (int i = 0; i < XPT; ++i) reinterpret_cast<uint4*>(xs)[tid + i * NW * 64] = xv[i];
      __syncthreads();
      staged = true;
    }
    fl_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
      const int g = wave + NW * i;
      if (g < G) unit_dot(w[i], sw[i], xs, g, m, acc);  // wave-uniform
    }
    if (lane < 16) part[wave * 16 + lane] = acc[0];
    __syncthreads();
    if (tid < 16) {
      float v = 0.0f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) v += part[ww * 16 + tid];
      y[rb * 16 + tid] = (uint16_t)f2bf(v);
    }
    __syncthreads();
  }
}

// Dequantisation through the same MFMA steps, bf16 [N, K] in row order (for the bit-exactness
// check against the reference's dequantisation): one wave per 1 KB unit.
__global__ __launch_bounds__(256) void k_dequant_tiled(const uint4* __restrict__ qt, const uint32_t* __restrict__ sz,
                                                       uint16_t* __restrict__ out, int n, int k) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 6;
  const int G = k >> 7;
  if (unit >= (int64_t)(n >> 4) * G) return;
  const int g = (int)(unit % G), rb = (int)(unit / G);
  const int b = lane >> 4, c = lane & 15;
  uint32_t o[8][2];
  unit_dq_t<8>(qt[unit * 64 + lane], sz[(size_t)(rb * 16 + c) * G + g], mx_lane(), o);
#pragma unroll
  for (int t = 0; t < 8; ++t)  // row c of the block, columns 16t + 4b .. +3 of group g
    *reinterpret_cast<uint2*>(out + (size_t)(rb * 16 + c) * k + g * 128 + 16 * t + 4 * b) = make_uint2(o[t][0], o[t][1]);
}

// Diagnostic: the compute rate of the exact dequantisation with an M = 8 matrix-core product and
// no memory traffic at all. Each wave keeps PDQ_NU units (16 rows x one 128-group: 2048 weights)
// of seeded pseudo-random words in registers and recomputes them `iters` times against 8 token
// rows in LDS -- k_verify's tile product at M = 8 with the weights already there. MODE 0: this
// library's row layout, dequantised on the vector ALUs (dq32, four 16x16x32 MFMAs per 32 weights:
// the verify tiles' former product, and fl_gemm_int4's); MODE 1: the tiled layout, both exact fp32 steps on 4x4x4 MFMAs and the
// dot on a 16x16x32 MFMA per two tiles (unit_mma_t over two tiles at a time); MODE 2: the same
// with each step batched over the unit's 8 tiles (unit_mma_t<8>, the kernels' form);
// MODES 3 / 4: M = 1 as the decode kernel computes it, one row-layout chunk per lane dotted with x
// on the vector ALUs, dequantised by dq32 (3) or by the lane-local matrix-core dq32_mx (4).
// out[2 wg] = the workgroup's 100 MHz ticks, out[2 wg + 1] = bits of its result (kept so the
// work is not dropped).
constexpr int PDQ_NU = 3, PDQ_LD = 392;  // units per wave; token-row pitch (bf16)
template <int MODE>
__global__ __launch_bounds__(512, 1) void k_probe_dequant(int iters, unsigned long long* __restrict__ out) {
  __shared__ __align__(16) uint16_t xs[17 * PDQ_LD];  // token rows 0..7, row 16 zero (rows 8..15)
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < 17 * PDQ_LD / 2; i += 512)
    reinterpret_cast<uint32_t*>(xs)[i] = i < 8 * PDQ_LD / 2 ? 0x3F803F80u ^ ((i * 2654435761u) & 0x007F007Fu) : 0u;
  __syncthreads();
  uint4 w[PDQ_NU];
  uint32_t s[PDQ_NU];
  uint32_t h = (blockIdx.x * 512u + tid) * 2654435761u + 12345u;
  auto next = [&h]() {
    h ^= h << 13;
    h ^= h >> 17;
    h ^= h << 5;
    return h;
  };
#pragma unroll
  for (int u = 0; u < PDQ_NU; ++u) {
    w[u] = make_uint4(next(), next(), next(), next());
    s[u] = 0x3A833A83u ^ (next() & 0x00070007u);  // scales near 1e-3, zeros near 1e-3
  }
  const int r = lane & 15, c = lane >> 4;
  fl_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const MxLane mxl = mx_lane();
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < PDQ_NU; ++u) {
      // the words are opaque to the compiler each pass, so nothing is hoisted out of the loop
      asm volatile("" : "+v"(w[u].x), "+v"(w[u].y), "+v"(w[u].z), "+v"(w[u].w), "+v"(s[u]));
      if constexpr (MODE == 0) {
        const uint16_t* xrow = xs + (r < 8 ? r : 16) * PDQ_LD + c * 32 + u * 128;
        uint4 xa[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) xa[e] = *reinterpret_cast<const uint4*>(xrow + e * 8);
        uint32_t d[4][4];
        dq32(w[u], dq_const(s[u]), d);
        mfma_chunk(d, xa, acc);
      } else if constexpr (MODE == 3 || MODE == 4) {
        // M = 1, decode's form: one row chunk per lane dotted with x on the vector ALUs
        const uint16_t* xrow = xs + c * 32 + u * 128;
        uint4 xa[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) xa[e] = *reinterpret_cast<const uint4*>(xrow + e * 8);
        uint32_t d[4][4];
        if constexpr (MODE == 3)
          dq32(w[u], dq_const(s[u]), d);
        else
          dq32_mx(w[u], s[u], mxl, d);
        float a = acc[0];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a = dot2_bf16(d[0][i], xa[i].x, a);
          a = dot2_bf16(d[1][i], xa[i].y, a);
          a = dot2_bf16(d[2][i], xa[i].z, a);
          a = dot2_bf16(d[3][i], xa[i].w, a);
        }
        acc[0] = a;
      } else if constexpr (MODE == 2) {
        const uint16_t* xrow = xs + (r < 8 ? r : 16) * PDQ_LD + u * 128 + 4 * c;
        unit_mma_t<8>(w[u], s[u], mxl, xrow, acc);
      } else {
        const uint16_t* xrow = xs + (r < 8 ? r : 16) * PDQ_LD + u * 128 + 4 * c;
        unit_mma_t<2>(w[u], s[u], mxl, xrow, acc);
      }
    }
  }
  const float v = acc[0] + acc[1] + acc[2] + acc[3];
  __syncthreads();  // the workgroup's time is its slowest wave's
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  if (tid == 0) {
    out[2 * blockIdx.x] = t1 - t0;
    out[2 * blockIdx.x + 1] = __float_as_uint(v);
  }
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

int fl_tile_int4(const uint32_t* q, uint32_t* qt, int32_t n, int32_t k, void* stream) {
  if (!q || !qt || n <= 0 || k <= 0 || (n % 16) != 0 || (k % FL_GROUP) != 0) return FL_E_ARG;
  const int64_t chunks = (int64_t)(n / 16) * (k / 128) * 64;
  const int64_t blocks = (chunks + 255) / 256;
  if (blocks > 0x7FFFFFFF) return FL_E_ARG;
  hipLaunchKernelGGL(k_tile_int4, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), q,
                     reinterpret_cast<uint4*>(qt), n, k);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

int fl_dequant_int4_tiled(const uint32_t* qt, const uint32_t* sz, uint16_t* out, int32_t n, int32_t k,
                          void* stream) {
  if (!qt || !sz || !out || n <= 0 || k <= 0 || (n % 16) != 0 || (k % FL_GROUP) != 0) return FL_E_ARG;
  const int64_t units = (int64_t)(n / 16) * (k / 128);
  const int64_t blocks = (units + 3) / 4;
  if (blocks > 0x7FFFFFFF) return FL_E_ARG;
  hipLaunchKernelGGL(k_dequant_tiled, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint4*>(qt), sz, out, n, k);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

int fl_gemv_int4_tiled(const uint32_t* qt, const uint32_t* sz, const uint16_t* x, uint16_t* y, int32_t n,
                       int32_t k, void* stream) {
  if (!qt || !sz || !x || !y || n <= 0 || k <= 0 || (n % 16) != 0 || (k % FL_GROUP) != 0 || k > 16384)
    return FL_E_ARG;
  const int G = k / FL_GROUP;
  const uint4* q4 = reinterpret_cast<const uint4*>(qt);
  // every unit of a wave in registers: 4 waves x 8 units (K <= 4096), 8 x 8 (K <= 8192); LDS: the
  // x slots (2 per thread) and the waves' partial sums
  if (G <= 32) {
    hipLaunchKernelGGL((k_gemv_tiled_pf<4, 8>), dim3(n / 16), dim3(4 * 64), (size_t)2 * 4 * 64 * 16 + 4 * 16 * 4,
                       as_stream(stream), q4, sz, x, y, n, k);
  } else if (G <= 64) {
    hipLaunchKernelGGL((k_gemv_tiled_pf<8, 8>), dim3(n / 16), dim3(8 * 64), (size_t)2 * 8 * 64 * 16 + 8 * 16 * 4,
                       as_stream(stream), q4, sz, x, y, n, k);
  } else {
    hipLaunchKernelGGL(k_gemv_tiled, dim3(n / 16), dim3(TW_NW * 64), (size_t)k * 2 + TW_NW * 16 * 4,
                       as_stream(stream), q4, sz, x, y, n, k);
  }
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

int fl_probe_dequant(int32_t mode, int32_t iters, uint64_t* out, int32_t* grid, void* stream) {
  if (mode < 0 || mode > 4 || iters < 1 || iters > 1000000 || !out || !grid) return FL_E_ARG;
  int dev = 0, cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu < 1)
    return FL_E_HIP;
  *grid = cu;
  auto* o = reinterpret_cast<unsigned long long*>(out);
  if (mode == 0)
    hipLaunchKernelGGL(k_probe_dequant<0>, dim3(cu), dim3(512), 0, as_stream(stream), (int)iters, o);
  else if (mode == 1)
    hipLaunchKernelGGL(k_probe_dequant<1>, dim3(cu), dim3(512), 0, as_stream(stream), (int)iters, o);
  else if (mode == 2)
    hipLaunchKernelGGL(k_probe_dequant<2>, dim3(cu), dim3(512), 0, as_stream(stream), (int)iters, o);
  else if (mode == 3)
    hipLaunchKernelGGL(k_probe_dequant<3>, dim3(cu), dim3(512), 0, as_stream(stream), (int)iters, o);
  else
    hipLaunchKernelGGL(k_probe_dequant<4>, dim3(cu), dim3(512), 0, as_stream(stream), (int)iters, o);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

}  // extern "C"
