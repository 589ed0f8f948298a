// Diagnostic micro-benchmark of one inter-workgroup hand-off: the latency of handing a tagged
// vector from every producer workgroup to every consumer workgroup inside one launch, as the
// decode and verify kernels do between phases (no grid barrier: consumers poll tagged words).
// No counterpart in the reference, which times its grid barrier in isolation instead
// (result.md:38-40).
//
// One workgroup of 512 threads per CU (the decode kernel's shape; the LDS request keeps it at one
// per CU). Round r: every producer stores its share of a `words`-word vector, each word a 16-bit
// value with tag r + 1 above it, then polls every word of the vector until all carry tag r + 1
// (device-coherent loads with a short sleep between polls, as the kernels' waits). Rounds
// alternate between two buffers, so a fast producer never overwrites a word that a slow consumer
// of the previous round still waits for. Each workgroup's time for `rounds` chained rounds,
// divided by rounds, is one hand-off (the exchange plus the poll's own round trip).
//
// Modes (a group = the workgroups that exchange one vector):
//   0: all workgroups; the uncached exchange memory of the decode kernel;
//   1: the workgroups of one XCD (blockIdx % 8: the round-robin dispatch over the 8 XCDs of an
//      MI355X), 8 independent groups; the same memory;
//   2: the workgroups of one XCD; ordinary device memory, whose coherent loads are served by
//      that XCD's L2 (the one L2 all the group's CUs share);
//   3: all workgroups, uncached memory, polled the way the decode kernel's waits poll: 16-byte
//      groups of 4 words, every missing group re-requested at once, 1 to 3 rounds of requests in
//      flight (k_probe_groups);
//   4: the workgroups of one XCD (as mode 1), polled as mode 3 with one round in flight.
// Modes 0-2 poll single words with a sleep between polls.
// Every workgroup also records its XCC_ID hardware register, so the host can check the
// blockIdx-to-XCD mapping that modes 1 and 2 assume. Every wait is bounded (about 0.5 s): a
// workgroup that is not resident, or a mapping that is not the assumed one, ends in a reported
// timeout, not a hang.
#include "fl_common.h"
#include <mutex>

namespace {

constexpr int PR_NT = 512;
constexpr int PR_GROUPS = 8;                          // XCDs of an MI355X
constexpr int PR_MAXW = 8192;                         // words per vector
constexpr int PR_LDS = 96 * 1024;                     // keeps one workgroup per CU
constexpr int PR_MAXP = PR_MAXW / PR_NT;              // words polled per thread, at most
constexpr unsigned long long PR_SPIN = 50000000ull;   // 0.5 s of the 100 MHz realtime clock

// out[2 * wg] = ticks of the rounds (100 MHz clock), out[2 * wg + 1] = XCC_ID | timed out << 32
__global__ __launch_bounds__(PR_NT, 1) void k_probe_handoff(uint32_t* __restrict__ buf, int words,
                                                            int rounds, int mode,
                                                            unsigned long long* __restrict__ out) {
  extern __shared__ uint32_t pad[];
  const int tid = threadIdx.x, wg = blockIdx.x, G = gridDim.x;
  const bool local = mode != 0;
  const int group = local ? wg % PR_GROUPS : 0;
  const int gsize = local ? (G - group + PR_GROUPS - 1) / PR_GROUPS : G;  // workgroups in the group
  const int gi = local ? wg / PR_GROUPS : wg;                            // index within it
  uint32_t* vec = buf + (size_t)group * 2 * words;                       // the group's two buffers
  const int share = (words + gsize - 1) / gsize;
  const int w0 = gi * share, w1 = min(words, w0 + share);
  if (tid == 0) pad[0] = 0;  // the LDS request only sets occupancy
  bool timed_out = false;
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int r = 0; r < rounds && !timed_out; ++r) {
    uint32_t* v = vec + (size_t)(r & 1) * words;
    const uint32_t tag = (uint32_t)(r % 65535) + 1u;
    // stored without waiting for them (the kernels' producers do not wait either: the tag in
    // every word is what the consumers check)
    for (int i = w0 + tid; i < w1; i += PR_NT) st_coh_u32(v + i, (tag << 16) | (uint32_t)(i & 0xFFFF));
    // poll: every thread requests its words, then re-requests the ones not yet tagged
    uint32_t got[PR_MAXP];
#pragma unroll
    for (int j = 0; j < PR_MAXP; ++j) {
      const int i = tid + j * PR_NT;
      got[j] = i < words ? ld_coh_u32(v + i) : (tag << 16);
    }
    const unsigned long long ts = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      bool done = true;
#pragma unroll
      for (int j = 0; j < PR_MAXP; ++j) done &= (got[j] >> 16) == tag;
      if (done) break;
      if (__builtin_amdgcn_s_memrealtime() - ts > PR_SPIN) {
        timed_out = true;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
#pragma unroll
      for (int j = 0; j < PR_MAXP; ++j) {
        const int i = tid + j * PR_NT;
        if ((got[j] >> 16) != tag) got[j] = ld_coh_u32(v + i);
      }
    }
    timed_out = __syncthreads_or(timed_out);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  if (tid == 0) {
    const uint32_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);  // hwreg(HW_REG_XCC_ID)
    out[2 * wg] = t1 - t0;
    out[2 * wg + 1] = (unsigned long long)xcc | ((unsigned long long)timed_out << 32);
  }
}

// Mode 3: all workgroups over the uncached exchange memory, polled in 16-byte groups of 4 words
// (the decode kernel's poll_issue form) with DEPTH rounds of requests in flight: round r + 1 is
// requested before round r's answers are checked, `gap` x 64 cycles after it, so a word that
// lands just after one round passed the coherence point is seen by the next without a full round
// trip in between. Each round re-requests only the groups not yet seen complete (complete groups
// get an out-of-range request, which touches no memory and keeps the requests branch-free),
// `resleep` x 64 cycles after the answers that found them incomplete. local: the groups of mode 4
// (each XCD's workgroups exchange a vector of their own, in buffers of their own).
constexpr int PR_MAXG = PR_MAXW / 4 / PR_NT;  // 16-byte groups polled per thread, at most
template <int DEPTH>
__global__ __launch_bounds__(PR_NT, 1) void k_probe_groups(uint32_t* __restrict__ buf, int words,
                                                           int rounds, int gap, int resleep, int local,
                                                           unsigned long long* __restrict__ out) {
  extern __shared__ uint32_t pad[];
  const int tid = threadIdx.x, wg = blockIdx.x, G = gridDim.x;
  const int group = local ? wg % PR_GROUPS : 0;
  const int gsize = local ? (G - group + PR_GROUPS - 1) / PR_GROUPS : G;  // workgroups in the group
  const int gi = local ? wg / PR_GROUPS : wg;                            // index within it
  uint32_t* const vec = buf + (size_t)group * 2 * words;                 // the group's two buffers
  const int share = (words + gsize - 1) / gsize;
  const int w0 = gi * share, w1 = min(words, w0 + share);
  const int ng = words >> 2;
  if (tid == 0) pad[0] = 0;
  bool timed_out = false;
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int r = 0; r < rounds && !timed_out; ++r) {
    uint32_t* v = vec + (size_t)(r & 1) * words;
    const uint32_t tag = (uint32_t)(r % 65535) + 1u;
    for (int i = w0 + tid; i < w1; i += PR_NT) st_coh_u32(v + i, (tag << 16) | (uint32_t)(i & 0xFFFF));
    const auto rs = buf_rsrc(v, (uint32_t)words * 4u);
    bool seen[PR_MAXG];
#pragma unroll
    for (int j = 0; j < PR_MAXG; ++j) seen[j] = tid + j * PR_NT >= ng;
    uint4 q[DEPTH][PR_MAXG];
    auto issue = [&](uint4 (&d)[PR_MAXG]) {
#pragma unroll
      for (int j = 0; j < PR_MAXG; ++j)
        d[j] = buf_ld128_coh(rs, seen[j] ? 0xFFFFFFF0u : (uint32_t)(tid + j * PR_NT) * 16u);
    };
    auto take = [&](const uint4 (&d)[PR_MAXG]) {
      bool all = true;
#pragma unroll
      for (int j = 0; j < PR_MAXG; ++j) {
        const uint4 w = d[j];
        seen[j] = seen[j] || (((w.x >> 16) == tag) & ((w.y >> 16) == tag) & ((w.z >> 16) == tag) &
                              ((w.w >> 16) == tag));
        all &= seen[j];
      }
      return all;
    };
    auto pause = [&] {
      for (int s = 0; s < gap; ++s) __builtin_amdgcn_s_sleep(1);
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      if (d) pause();
      issue(q[d]);
    }
    const unsigned long long ts = __builtin_amdgcn_s_memrealtime();
    for (bool done = false; !done;) {
#pragma unroll
      for (int d = 0; d < DEPTH && !done; ++d) {
        if (take(q[d])) {
          done = true;
        } else {
          for (int t = 0; t < resleep; ++t) __builtin_amdgcn_s_sleep(1);
          issue(q[d]);
        }
      }
      if (!done && __builtin_amdgcn_s_memrealtime() - ts > PR_SPIN) {
        timed_out = true;
        break;
      }
    }
    timed_out = __syncthreads_or(timed_out);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  if (tid == 0) {
    const uint32_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);  // hwreg(HW_REG_XCC_ID)
    out[2 * wg] = t1 - t0;
    out[2 * wg + 1] = (unsigned long long)xcc | ((unsigned long long)timed_out << 32);
  }
}

// exchange buffers, kept for the process (the uncached one must never be freed once read)
std::mutex g_probe_mu;
uint32_t* g_probe_uc[64] = {};
uint32_t* g_probe_rw[64] = {};

}  // namespace

extern "C" {

int fl_probe_handoff(int32_t mode, int32_t words, int32_t rounds, uint64_t* out, int32_t* grid,
                     void* stream) {
  // mode: bits 0-7 the kind (0..4); kind 3 also takes the poll depth (bits 8-11, 1..3), the gap
  // between the first rounds' requests (bits 16-23, x 64 cycles) and the sleep before a re-request
  // (bits 24-30, x 64 cycles); kind 4 takes none (one round in flight)
  const int kind = mode & 0xFF, gap = (mode >> 16) & 0xFF, resleep = (mode >> 24) & 0x7F;
  const int depth = kind == 4 ? 1 : (mode >> 8) & 0xF;
  if (mode < 0 || kind > 4 || (kind != 3 && mode != kind) || (kind >= 3 && (depth < 1 || depth > 3 || words % 4)) ||
      words < 4 || words > PR_MAXW || rounds < 1 || rounds > 100000 || !out || !grid)
    return FL_E_ARG;
  const int local = kind == 4;
  int dev = 0, cu = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return FL_E_HIP;
  if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return FL_E_HIP;
  const size_t bytes = (size_t)PR_GROUPS * 2 * PR_MAXW * 4;
  uint32_t* buf;
  {
    std::lock_guard<std::mutex> lk(g_probe_mu);
    uint32_t** slot = kind == 2 ? &g_probe_rw[dev] : &g_probe_uc[dev];
    if (!*slot) {
      void* p = nullptr;
      const hipError_t e = kind == 2 ? hipMalloc(&p, bytes) : hipExtMallocWithFlags(&p, bytes, hipDeviceMallocUncached);
      if (e != hipSuccess) return FL_E_HIP;
      if (hipMemset(p, 0, bytes) != hipSuccess) return FL_E_HIP;
      *slot = reinterpret_cast<uint32_t*>(p);
    }
    buf = *slot;
  }
  const void* kfn = kind < 3 ? reinterpret_cast<const void*>(k_probe_handoff)
                  : depth == 1 ? reinterpret_cast<const void*>(k_probe_groups<1>)
                  : depth == 2 ? reinterpret_cast<const void*>(k_probe_groups<2>)
                               : reinterpret_cast<const void*>(k_probe_groups<3>);
  // every workgroup must be resident at once (one per CU)
  int occ = 0;
  if (hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, PR_LDS) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kfn, PR_NT, PR_LDS) != hipSuccess || occ < 1)
    return FL_E_LAUNCH;
  // tags restart at 1 each call: clear both buffers of every group first (stream-ordered)
  if (hipMemsetAsync(buf, 0, bytes, reinterpret_cast<hipStream_t>(stream)) != hipSuccess) return FL_E_HIP;
  *grid = cu;
  auto* o = reinterpret_cast<unsigned long long*>(out);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (kind < 3)
    hipLaunchKernelGGL(k_probe_handoff, dim3(cu), dim3(PR_NT), PR_LDS, s, buf, (int)words, (int)rounds, kind, o);
  else if (depth == 1)
    hipLaunchKernelGGL(k_probe_groups<1>, dim3(cu), dim3(PR_NT), PR_LDS, s, buf, (int)words, (int)rounds, gap, resleep,
                       local, o);
  else if (depth == 2)
    hipLaunchKernelGGL(k_probe_groups<2>, dim3(cu), dim3(PR_NT), PR_LDS, s, buf, (int)words, (int)rounds, gap, resleep,
                       local, o);
  else
    hipLaunchKernelGGL(k_probe_groups<3>, dim3(cu), dim3(PR_NT), PR_LDS, s, buf, (int)words, (int)rounds, gap, resleep,
                       local, o);
  return hipGetLastError() == hipSuccess ? FL_OK : FL_E_LAUNCH;
}

}  // extern "C"
