// Device helpers shared by all flint_amd kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/flint_amd.h"

typedef __bf16 fl_bf16x2 __attribute__((ext_vector_type(2)));

#define FL_WAVE 64

// ---- bf16 <-> fp32 (round-to-nearest-even, the rounding torch uses for every bf16 op) ----
__device__ __forceinline__ float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }
__device__ __forceinline__ float bflo(uint32_t pk) { return __uint_as_float(pk << 16); }
__device__ __forceinline__ float bfhi(uint32_t pk) { return __uint_as_float(pk & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t f2bf(float f) {
  __bf16 b = (__bf16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  fl_bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
// value of f after rounding to bf16
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(fl_bf16x2, a),
                                         __builtin_bit_cast(fl_bf16x2, b), c, false);
}

// ---- int4 group dequantisation -------------------------------------------------------------
// One packed word holds 8 consecutive elements, element e at bits 4e. Produces the four
// packed bf16 pairs (e0,e1) (e2,e3) (e4,e5) (e6,e7) of
//     dq = bf16( bf16((q - 8) * s) + z )
// i.e. gpt-fast's group_dequantize_tensor_from_qparams (reference engine/quantize.py:152-154):
// int32.sub(8).mul(bf16 scale) rounds to bf16, then .add(bf16 zero) rounds to bf16 again.
// (q-8)*s has at most 12 significant bits, so fma(q, s, -8s) is exact in fp32.
__device__ __forceinline__ void dq8(uint32_t w, float s, float z, float c8, uint32_t out[4]) {
  const uint32_t lo = w & 0x0F0F0F0Fu;
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float q0 = (float)((lo >> (8 * b)) & 0xFFu);
    const float q1 = (float)((hi >> (8 * b)) & 0xFFu);
    const uint32_t p = pack_bf16x2(__builtin_fmaf(q0, s, c8), __builtin_fmaf(q1, s, c8));
    out[b] = pack_bf16x2(bflo(p) + z, bfhi(p) + z);
  }
}

// dot of one 16-byte chunk (32 int4 elements of one 128-group) with 32 bf16 x values
// (16 packed pairs), accumulated into acc.
__device__ __forceinline__ float chunk_dot(const uint4 w, uint32_t szw, const uint4* x4, float acc) {
  const float s = bf2f(szw & 0xFFFFu), z = bf2f(szw >> 16), c8 = -8.0f * s;
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t d[4];
    dq8(ws[j], s, z, c8, d);
    const uint4 xv = x4[j];
    acc = dot2_bf16(d[0], xv.x, acc);
    acc = dot2_bf16(d[1], xv.y, acc);
    acc = dot2_bf16(d[2], xv.z, acc);
    acc = dot2_bf16(d[3], xv.w, acc);
  }
  return acc;
}

// ---- wave reductions (wave64) ---------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// sum over aligned groups of `width` lanes (width a power of two <= 64); fixed order
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---- argmax key: larger key = larger value, then smaller index --------------------------------
__device__ __forceinline__ unsigned long long amax_key(float v, uint32_t idx) {
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ uint32_t amax_index(unsigned long long key) {
  return 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull);
}
__device__ __forceinline__ unsigned long long u64max(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    unsigned long long u = __shfl_xor(v, o, 64);
    v = u64max(v, u);
  }
  return v;
}

// SiLU as torch computes it for a bf16 tensor: x / (1 + exp(-x)) in fp32.
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
