// Device helpers shared by all flint_amd kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/flint_amd.h"

typedef __bf16 fl_bf16x2 __attribute__((ext_vector_type(2)));
typedef float fl_f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 fl_bf16x8 __attribute__((ext_vector_type(8)));

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
// Packed word layout (8 consecutive elements e0..e7 of one row): element 2k sits in nibble k and
// element 2k+1 in nibble k+4 (k = 0..3), i.e. bits 4k and 16+4k. One AND-OR then yields the
// bf16 pair (128 + q_2k, 128 + q_2k+1) (0x4300 = 128.0, the nibble lands in the mantissa).
//
// dq = bf16( bf16((q - 8) * s) + z ) is gpt-fast's group_dequantize_tensor_from_qparams
// (reference engine/quantize.py:152-154): int32.sub(8).mul(bf16 scale) rounds to bf16, then
// .add(bf16 zero) rounds to bf16 again. Both fp32 steps run on v_dot2_f32_bf16, whose bf16
// products are exact in fp32:
//   (128+q)*s + 0 + (-136*s) = (q-8)*s          exact ((q-8)*s has <= 12 significant bits)
//   p_bf16*1 + 0 + z          = fp32(p_bf16 + z) one rounding, as torch's fp32 add
// and v_cvt_pk_bf16_f32 rounds each result to bf16 (RNE). 35 VALU ops per 8 weights.
struct DqConst {
  uint32_t s_lo, s_hi;  // bf16 pairs (s, 0) and (0, s)
  float c;              // -136 * s (exact)
  float z;
};
__device__ __forceinline__ DqConst dq_const(uint32_t szw) {
  const uint32_t sb = szw & 0xFFFFu;
  DqConst k;
  k.s_lo = sb;
  k.s_hi = sb << 16;
  k.c = -136.0f * bf2f(sb);
  k.z = bf2f(szw >> 16);
  return k;
}

// One step (nibbles 0 and 4, i.e. bits 0-3 and 16-19) of four words w0..w3 of one 128-group:
// o[i] = packed bf16 dequantised pair of word i. SHIFT first moves the words right by 4 in place,
// so consecutive steps walk the nibble pairs 0..3 of the same running words (no copy of the
// original words is kept, which a shift by 4j from the original would need). One asm block so the instruction order is
// fixed: the three-address (VOP3P) v_dot2_f32_bf16 needs no copy of its shared accumulator, and
// the order puts at least three instructions between every write and its first read (a dot
// reading a VGPR written just before it, and any read of a dot's result right after the dot,
// need wait states that the compiler does not insert across inline asm), so the block needs no
// s_nop of its own. It ends with two wait states, so the outputs may feed an MFMA or a VOP3P
// instruction right away (the compiler sees no VALU write inside the asm).
template <bool SHIFT>
__device__ __forceinline__ void dq_step4(uint32_t& w0, uint32_t& w1, uint32_t& w2, uint32_t& w3,
                                         const DqConst& k, uint32_t magic, uint32_t one_lo,
                                         uint32_t one_hi, uint32_t (&o)[4]) {
  uint32_t m0, m1, m2, m3, p00, p01, p10, p11, p20, p21, p30, p31, p0, p1, p2, p3;
  uint32_t d00, d01, d10, d11, d20, d21, d30, d31;
  if (SHIFT) {
    asm("v_lshrrev_b32 %0, 4, %0\n\t"
        "v_lshrrev_b32 %1, 4, %1\n\t"
        "v_lshrrev_b32 %2, 4, %2\n\t"
        "v_lshrrev_b32 %3, 4, %3"
        : "+v"(w0), "+v"(w1), "+v"(w2), "+v"(w3));
  }
  asm("v_and_or_b32 %[m0], %[w0], %[mask], %[magic]\n\t"
      "v_and_or_b32 %[m1], %[w1], %[mask], %[magic]\n\t"
      "v_and_or_b32 %[m2], %[w2], %[mask], %[magic]\n\t"
      "v_and_or_b32 %[m3], %[w3], %[mask], %[magic]\n\t"
      "v_dot2_f32_bf16 %[p00], %[m0], %[slo], %[c]\n\t"
      "v_dot2_f32_bf16 %[p10], %[m1], %[slo], %[c]\n\t"
      "v_dot2_f32_bf16 %[p01], %[m0], %[shi], %[c]\n\t"
      "v_dot2_f32_bf16 %[p11], %[m1], %[shi], %[c]\n\t"
      "v_dot2_f32_bf16 %[p20], %[m2], %[slo], %[c]\n\t"
      "v_dot2_f32_bf16 %[p30], %[m3], %[slo], %[c]\n\t"
      "v_dot2_f32_bf16 %[p21], %[m2], %[shi], %[c]\n\t"
      "v_dot2_f32_bf16 %[p31], %[m3], %[shi], %[c]\n\t"
      "v_cvt_pk_bf16_f32 %[p0], %[p00], %[p01]\n\t"
      "v_cvt_pk_bf16_f32 %[p1], %[p10], %[p11]\n\t"
      "v_cvt_pk_bf16_f32 %[p2], %[p20], %[p21]\n\t"
      "v_cvt_pk_bf16_f32 %[p3], %[p30], %[p31]\n\t"
      "v_dot2_f32_bf16 %[d00], %[p0], %[olo], %[z]\n\t"
      "v_dot2_f32_bf16 %[d10], %[p1], %[olo], %[z]\n\t"
      "v_dot2_f32_bf16 %[d01], %[p0], %[ohi], %[z]\n\t"
      "v_dot2_f32_bf16 %[d11], %[p1], %[ohi], %[z]\n\t"
      "v_dot2_f32_bf16 %[d20], %[p2], %[olo], %[z]\n\t"
      "v_dot2_f32_bf16 %[d30], %[p3], %[olo], %[z]\n\t"
      "v_dot2_f32_bf16 %[d21], %[p2], %[ohi], %[z]\n\t"
      "v_dot2_f32_bf16 %[d31], %[p3], %[ohi], %[z]\n\t"
      "v_cvt_pk_bf16_f32 %[o0], %[d00], %[d01]\n\t"
      "v_cvt_pk_bf16_f32 %[o1], %[d10], %[d11]\n\t"
      "v_cvt_pk_bf16_f32 %[o2], %[d20], %[d21]\n\t"
      "v_cvt_pk_bf16_f32 %[o3], %[d30], %[d31]\n\t"
      "s_nop 1"
      : [m0] "=&v"(m0), [m1] "=&v"(m1), [m2] "=&v"(m2), [m3] "=&v"(m3),
        [p00] "=&v"(p00), [p01] "=&v"(p01), [p10] "=&v"(p10), [p11] "=&v"(p11),
        [p20] "=&v"(p20), [p21] "=&v"(p21), [p30] "=&v"(p30), [p31] "=&v"(p31),
        [p0] "=&v"(p0), [p1] "=&v"(p1), [p2] "=&v"(p2), [p3] "=&v"(p3),
        [d00] "=&v"(d00), [d01] "=&v"(d01), [d10] "=&v"(d10), [d11] "=&v"(d11),
        [d20] "=&v"(d20), [d21] "=&v"(d21), [d30] "=&v"(d30), [d31] "=&v"(d31),
        [o0] "=&v"(o[0]), [o1] "=&v"(o[1]), [o2] "=&v"(o[2]), [o3] "=&v"(o[3])
      : [w0] "v"(w0), [w1] "v"(w1), [w2] "v"(w2), [w3] "v"(w3), [mask] "s"(0x000F000Fu),
        [magic] "v"(magic), [slo] "v"(k.s_lo), [shi] "v"(k.s_hi), [c] "v"(k.c),
        [olo] "v"(one_lo), [ohi] "v"(one_hi), [z] "v"(k.z));
}

// Dequantise the four words of a 16-byte chunk (32 elements of one group):
// d[j][i] = packed pair (element 2j, 2j+1) of word i.
__device__ __forceinline__ void dq32(const uint4 w, const DqConst& k, uint32_t (&d)[4][4]) {
  const uint32_t magic = 0x43004300u;  // bf16 pair (128, 128)
  const uint32_t one_lo = 0x00003F80u, one_hi = 0x3F800000u;  // bf16 pairs (1, 0), (0, 1)
  uint32_t a = w.x, b = w.y, c = w.z, e = w.w;  // running words, shifted by 4 per step
  dq_step4<false>(a, b, c, e, k, magic, one_lo, one_hi, d[0]);
  dq_step4<true>(a, b, c, e, k, magic, one_lo, one_hi, d[1]);
  dq_step4<true>(a, b, c, e, k, magic, one_lo, one_hi, d[2]);
  dq_step4<true>(a, b, c, e, k, magic, one_lo, one_hi, d[3]);
}

// ---- the same dequantisation on 4x4x4 matrix-core steps, lane by lane --------------------------
// v_mfma_f32_4x4x4_16b_bf16 runs 16 independent 4x4x4 products, block b on lanes 4b..4b+3:
// row i of A comes from lane 4b + i and column j of B from lane 4b + j (their 4 bf16 along k),
// and lane 4b + j receives column j of D (its 4 fp32 along i) (checked on the GPU). With B = a
// lane's own 4 values and A = diag(s) (lane 4b + i puts s at k = i), lane j receives s * B_j[i]
// in slot i: an elementwise product, exact for bf16 inputs, with C added once. So
//   D1 = diag(s) . (128 + q) + (-136 s)  = (q - 8) s exactly (one nonzero product, as in dq_step4),
//   D2 = I . bf16(D1) + z               = fp32(bf16(D1) + z), the reference's fp32 add,
// each rounded to bf16 by v_cvt_pk_bf16_f32: the same bits as dq32, in 16 matrix-core steps and
// 28 vector instructions (plus the per-group constants) per 32 weights instead of 124. The
// diagonal is lane 4b + i's own scale, so the four lanes of every block must hold chunks with the
// same (scale, zero) word -- 4 consecutive lanes on 4 chunks of one 128-group of one row -- and
// all 64 lanes must run it together (wave-uniform control flow).
typedef short fl_s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ fl_s16x4 mx_s4(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(fl_s16x4, make_uint2(lo, hi));
}
struct MxLane {      // this lane's diagonal slot (lane & 3) as masks over the 4 bf16 of an operand
  uint32_t mlo, mhi;
  uint32_t mask, magic;  // the AND-OR constants, kept in registers (see mx_lane)
};
__device__ __forceinline__ MxLane mx_lane() {
  const int i = (int)(__lane_id() & 3);
  MxLane m;
  m.mlo = i == 0 ? 0x0000FFFFu : (i == 1 ? 0xFFFF0000u : 0u);
  m.mhi = i == 2 ? 0x0000FFFFu : (i == 3 ? 0xFFFF0000u : 0u);
  // (w & mask) | magic with both constants opaque to constant folding: the compiler emits one
  // v_and_or_b32 and, seeing the instruction, keeps the wait states the matrix-core results
  // around it need (an and-or written as inline asm would hide them from it)
  m.mask = 0x000F000Fu;
  m.magic = 0x43004300u;
  asm volatile("" : "+v"(m.mask));
  asm volatile("" : "+v"(m.magic));
  return m;
}
__device__ __forceinline__ void dq32_mx(const uint4 w, uint32_t szw, const MxLane& m, uint32_t (&d)[4][4]) {
  const uint32_t sb = szw & 0xFFFFu, sp = sb | (sb << 16);
  const fl_s16x4 as = mx_s4(sp & m.mlo, sp & m.mhi);
  const fl_s16x4 ai = mx_s4(0x3F803F80u & m.mlo, 0x3F803F80u & m.mhi);  // bf16 1.0 on the diagonal
  const float c1v = -136.0f * bf2f(sb), zv = bf2f(szw >> 16);
  const fl_f32x4 c1 = {c1v, c1v, c1v, c1v}, c2 = {zv, zv, zv, zv};
  uint32_t v[4] = {w.x, w.y, w.z, w.w};
  fl_f32x4 t[8];  // t[2j + h]: nibble step j of words 2h, 2h + 1
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t r0 = (v[2 * h] & m.mask) | m.magic, r1 = (v[2 * h + 1] & m.mask) | m.magic;
      t[2 * j + h] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(as, mx_s4(r0, r1), c1, 0, 0, 0);
    }
    if (j < 3) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] >>= 4;
    }
  }
  uint32_t a[8][2];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    a[u][0] = pack_bf16x2(t[u][0], t[u][1]);
    a[u][1] = pack_bf16x2(t[u][2], t[u][3]);
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) t[u] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(ai, mx_s4(a[u][0], a[u][1]), c2, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      d[j][2 * h] = pack_bf16x2(t[2 * j + h][0], t[2 * j + h][1]);
      d[j][2 * h + 1] = pack_bf16x2(t[2 * j + h][2], t[2 * j + h][3]);
    }
  }
}

// ---- the same on the tiled layout (fl_tile_int4): four rows of one column per lane ----------
// Lane L's 16 bytes of a 1 KB unit (16 rows x one 128-group) hold rows 4p..4p+3, p = (L / 4) % 4,
// at columns c + 16t, c = 4 (L / 16) + L % 4, t = 0..7 (tile t: words 0 / 1 rows 4p, 4p+1 at bits
// 4(t%4), 16 + 4(t%4) for t < 4 / t >= 4; words 2 / 3 rows 4p+2, 4p+3). Per tile, the 4x4x4 block
// of lanes 4b..4b+3 is a transpose: D1 = A . diag(s) + C1 with A = the lane's (128 + q) of four
// rows and B = diag(s of row L % 16 in slot L % 4), so lane L receives row L % 16 at columns
// 4 (L / 16) + 0..3 times its own row's scale; D2 = I . t + z as in dq32_mx. o[t] = the bf16 pairs
// (columns 4 (L / 16) + 0,1 / + 2,3 of tile t) of row L % 16, the B fragment of a 16x16x32 dot
// over tiles t, t + 1. The steps run NB tiles at a time (NB = 8: every rounding waits on an MFMA
// issued 8 instructions earlier).
template <int NB>
__device__ __forceinline__ void unit_dq_t(const uint4 w, uint32_t szw, const MxLane& m, uint32_t (&o)[8][2]) {
  static_assert(NB == 2 || NB == 4 || NB == 8, "tiles per batch");
  const uint32_t sb = szw & 0xFFFFu, sp = sb | (sb << 16);
  const fl_s16x4 bs = mx_s4(sp & m.mlo, sp & m.mhi);
  const fl_s16x4 ai = mx_s4(0x3F803F80u & m.mlo, 0x3F803F80u & m.mhi);
  const float c1v = -136.0f * bf2f(sb), zv = bf2f(szw >> 16);
  const fl_f32x4 c1 = {c1v, c1v, c1v, c1v}, c2 = {zv, zv, zv, zv};
  uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int t0 = 0; t0 < 8; t0 += NB) {
    fl_f32x4 d[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int t = t0 + u;
      const uint32_t lo = v[t >> 2] >> (4 * (t & 3)), hi = v[2 + (t >> 2)] >> (4 * (t & 3));
      d[u] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(mx_s4((lo & m.mask) | m.magic, (hi & m.mask) | m.magic),
                                                    bs, c1, 0, 0, 0);
    }
    uint32_t a[NB][2];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      a[u][0] = pack_bf16x2(d[u][0], d[u][1]);
      a[u][1] = pack_bf16x2(d[u][2], d[u][3]);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) d[u] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(ai, mx_s4(a[u][0], a[u][1]), c2, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      o[t0 + u][0] = pack_bf16x2(d[u][0], d[u][1]);
      o[t0 + u][1] = pack_bf16x2(d[u][2], d[u][3]);
    }
  }
}
// acc += X . dq^T over one tiled unit: xr = this lane's activation row (token L % 16, or a zero
// row) at the unit's group, plus 4 (L / 16); the 16x16x32 dot of tiles 2tp, 2tp + 1 takes x at
// columns 32tp + 4 (L / 16) + 0..3 and 32tp + 16 + 4 (L / 16) + 0..3 (its k = 8 (L / 16) + e).
// acc: lane L holds row L % 16 for tokens 4 (L / 16) + 0..3.
template <int NB>
__device__ __forceinline__ void unit_mma_t(const uint4 w, uint32_t szw, const MxLane& m, const uint16_t* xr,
                                           fl_f32x4& acc) {
  uint32_t o[8][2];
  unit_dq_t<NB>(w, szw, m, o);
#pragma unroll
  for (int tp = 0; tp < 4; ++tp) {
    const uint2 xa = *reinterpret_cast<const uint2*>(xr + 32 * tp);
    const uint2 xb = *reinterpret_cast<const uint2*>(xr + 32 * tp + 16);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(fl_bf16x8, make_uint4(xa.x, xa.y, xb.x, xb.y)),
        __builtin_bit_cast(fl_bf16x8, make_uint4(o[2 * tp][0], o[2 * tp][1], o[2 * tp + 1][0], o[2 * tp + 1][1])),
        acc, 0, 0, 0);
  }
}

// dot of one 16-byte chunk (32 int4 elements of one 128-group) with 32 bf16 x values (16 packed
// pairs), accumulated into acc; the chunk dequantised by dq32_mx (the four lanes of every 4-lane
// block on one 128-group of one row, all lanes together)
__device__ __forceinline__ float chunk_dot_mx(const uint4 w, uint32_t szw, const uint4* x4, float acc) {
  const uint4 x[4] = {x4[0], x4[1], x4[2], x4[3]};
  uint32_t d[4][4];
  dq32_mx(w, szw, mx_lane(), d);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = dot2_bf16(d[0][i], x[i].x, acc);
    acc = dot2_bf16(d[1][i], x[i].y, acc);
    acc = dot2_bf16(d[2][i], x[i].z, acc);
    acc = dot2_bf16(d[3][i], x[i].w, acc);
  }
  return acc;
}

// ---- int4 x bf16 on the matrix cores (M <= 16 activation rows) --------------------------------
// v_mfma_f32_16x16x32_bf16 lane layout (wave64): A fragment of lane l = row l%16, k (l/16)*8..+8;
// B fragment = column l%16, the same k; result D = column l%16, rows (l/16)*4 + 0..3.
// One 16-byte chunk (4 packed words = 32 weights of one 128-group) feeds four MFMA steps: lane
// (r = l%16, c = l/16) holds chunk c of group u of weight row r, and MFMA step e contracts the
// 32 k-values {128u + 32c + 8e + t}, so word e of the chunk is the B fragment and the matching
// 16 bytes of each activation row the A fragment (a permuted k order; every k appears once).

// acc += X(rows, the chunk's 32 k) . W(this lane's row, same k)^T; d from dq32, xa[e] = 8 bf16
// of this lane's activation row at k = 128u + 32c + 8e
__device__ __forceinline__ void mfma_chunk(const uint32_t (&d)[4][4], const uint4 (&xa)[4],
                                           fl_f32x4& acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint4 bw = make_uint4(d[0][e], d[1][e], d[2][e], d[3][e]);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(fl_bf16x8, xa[e]),
                                                  __builtin_bit_cast(fl_bf16x8, bw), acc, 0, 0, 0);
  }
}

// nibble position of element e (0..7) within its packed word
__device__ __forceinline__ int nib_pos(int e) { return (e >> 1) + 4 * (e & 1); }

// ---- device-coherent accesses ----------------------------------------------------------------
// Data exchanged between workgroups inside one launch goes through agent-scope relaxed atomic
// loads/stores (global_load/store ... sc1: coherent across the 8 XCD L2s) instead of plain
// accesses plus acquire/release fences, which on gfx950 write back / invalidate a whole L2.
__device__ __forceinline__ void st_coh_u16(uint16_t* p, uint32_t v) {
  __hip_atomic_store(p, (uint16_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh_f32(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_coh_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh_f32(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 ld_coh_u128(const void* p) {
  unsigned long long* q = reinterpret_cast<unsigned long long*>(const_cast<void*>(p));
  const unsigned long long a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
}
__device__ __forceinline__ void st_coh_u64(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_coh_u64(const unsigned long long* p) {
  return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
// ---- range-checked loads ----------------------------------------------------------------------
// A raw buffer resource over [base, base + bytes): loads at offsets past the end return 0 and
// touch no memory. Prefetch loops use them instead of `if (in range) load`, which keeps them
// branch-free so the compiler can count outstanding loads exactly (a load issued under a branch
// makes later waits conservative: wait-for-all instead of wait-for-the-older-ones).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);  // raw buffer, 32-bit data format
}
__device__ __forceinline__ uint4 buf_ld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t buf_ld32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint2 buf_ld64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
// device-coherent variant (sc1: served past the non-coherent per-XCD L2s, like an agent-scope
// relaxed atomic load); each aligned dword of the result is read atomically
__device__ __forceinline__ uint4 buf_ld128_coh(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));
}
__device__ __forceinline__ uint2 buf_ld64_coh(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16));
}

// Workgroup barrier that orders LDS accesses only. __syncthreads also waits for every global
// load and store the wave has in flight (prefetched weights, published activations); this one
// does not, so a barrier between LDS producers and consumers never stalls on HBM traffic.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// wait until every memory operation this wave issued has completed (stores acknowledged at
// device scope); required before signalling other workgroups.
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0); }

// ---- cross-lane exchanges (wave64, VALU only) -------------------------------------------------
// __shfl_xor lowers to ds_bpermute, an LDS round trip per step. These use DPP lane patterns
// (within a 16-lane row) and gfx950's v_permlane16/32_swap (across rows) instead: one VALU op
// each. Every helper returns, in lane i, the value of lane i ^ mask.
// (every pattern used reads a valid lane, so the "old" operand is never selected; passing 0 lets
// the compiler fold the move into the consuming add / max as one DPP instruction)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_xor1(float v) { return dpp_f<0xB1>(v); }   // quad_perm 1,0,3,2
__device__ __forceinline__ float lane_xor2(float v) { return dpp_f<0x4E>(v); }   // quad_perm 2,3,0,1
__device__ __forceinline__ float lane_xor8(float v) { return dpp_f<0x128>(v); }  // row_ror:8
__device__ __forceinline__ float lane_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  // r[0]: odd rows replaced by the even rows below them, r[1]: even rows by the odd rows above
  return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}
// v(i) + v(i ^ 16) and v(i) + v(i ^ 32) (and max): both swap results are the lane pair, so
// one add gives the pair total in both lanes without a select
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// lane 7 - i within each group of 8 (after a 4-lane all-reduce, the other half's value)
__device__ __forceinline__ float lane_half_mirror(float v) { return dpp_f<0x141>(v); }
// lane 15 - i within each row of 16 (after an 8-lane all-reduce, the other half's value)
__device__ __forceinline__ float lane_mirror(float v) { return dpp_f<0x140>(v); }

// all-reduce over aligned groups of `width` lanes (width a power of two <= 64, wave-uniform).
// Every lane of a group ends with the bit-identical result (each step adds two values whose
// operands are the same pair in every lane). Fixed order.
__device__ __forceinline__ float group_sum(float v, int width) {
  if (width >= 2) v += lane_xor1(v);
  if (width >= 4) v += lane_xor2(v);
  if (width >= 8) v += lane_half_mirror(v);
  if (width >= 16) v += lane_mirror(v);
  if (width >= 32) v = xor16_sum(v);
  if (width >= 64) v = xor32_sum(v);
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  v += lane_xor1(v);
  v += lane_xor2(v);
  v += lane_half_mirror(v);
  v += lane_mirror(v);
  v = xor16_sum(v);
  return xor32_sum(v);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, lane_xor1(v));
  v = fmaxf(v, lane_xor2(v));
  v = fmaxf(v, lane_half_mirror(v));
  v = fmaxf(v, lane_mirror(v));
  v = xor16_max(v);
  return xor32_max(v);
}
// sum over the 8 lanes of a group of 8 (lanes 8a .. 8a+7)
__device__ __forceinline__ float sum8(float v) {
  v += lane_xor1(v);
  v += lane_xor2(v);
  return v + lane_half_mirror(v);
}
// sum / max over the lanes that share bits 0..2 of the lane id (lane i, i^8, ..., i^56)
__device__ __forceinline__ float sum_stride8(float v) {
  v += lane_xor8(v);
  v = xor16_sum(v);
  return xor32_sum(v);
}
__device__ __forceinline__ float max_stride8(float v) {
  v = fmaxf(v, lane_xor8(v));
  v = xor16_max(v);
  return xor32_max(v);
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

// ---- sampling helpers (used by the sampler and by the decode kernel's fused sampling) ----------
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


// SiLU of a bf16 tensor's element (torch: x / (1 + exp(-x)) in fp32), as x * sigmoid(x) with the
// hardware exp2 and reciprocal: within a few fp32 ulp of that (callers round the result to bf16),
// and the same -0 / x at the extremes
__device__ __forceinline__ float silu_f(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}
