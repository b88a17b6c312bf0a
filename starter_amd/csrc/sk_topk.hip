// sk_topk.hip - exact argmax plus approximate top-k over bf16 logits in one
// bandwidth-bound pass (engine/kernels/topk.py:17-46).
//
// The reference's algorithm, restated: 2048 "lanes" sweep the row with stride
// 2048; lane j keeps the largest value it sees at columns j, j + 2048, ...
// (strictly larger replaces, so the first occurrence of a value wins its lane)
// and its column.  Rank k of the output is then the largest remaining lane
// maximum, the lowest column among lanes holding it, and that lane is removed.
// Rank 0 is the exact argmax with torch's lowest-index tie rule; ranks >= 1
// miss a true top-k value only when two of them share a lane.
//
// MI355X mapping: one workgroup of 1024 threads per row, four sweep groups of
// 256.  Thread t of a group owns lanes 8t .. 8t+7, so one 16-byte load per
// thread reads 1 KiB contiguous per wave; group g takes the sweep steps
// g, g + 4, g + 8, ... and issues up to 20 of them before using any, so a
// row of the Qwen3 vocabulary (75 steps, 297 KiB) is requested in one round.  A group keeps, per
// lane, the largest value of its steps and the first column holding it; the
// four groups are merged per lane (larger value, then lower column), which is
// the single sweep's result: within a lane a later column replaces only a
// strictly larger value, i.e. the first occurrence of the lane maximum wins.
// The final selection is K rounds of a one-wave (max value, min column)
// reduction over the merged lane maxima.
#include "starter_amd.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include "sk_kernels.hpp"

namespace sk {

constexpr int TOPK_LANES = 2048;   // the reference's BLOCK
constexpr int TOPK_THREADS = 256;  // one sweep group
constexpr int TOPK_GROUPS = 4;     // sweep groups per row
constexpr int TOPK_UNROLL = 20;    // sweep steps a thread requests together
constexpr int TOPK_PER_THREAD = TOPK_LANES / TOPK_THREADS;   // 8 lanes per thread
constexpr int TOPK_MAX_K = 64;

__global__ void __launch_bounds__(TOPK_THREADS * TOPK_GROUPS)
topk_kernel(const uint16_t* __restrict__ L, int64_t ld, int V, int K, int vec, float* __restrict__ vals,
            int32_t* __restrict__ idxs) {
  __shared__ float s_gv[TOPK_GROUPS - 1][TOPK_LANES];   // lane maxima of groups 1..3
  __shared__ int s_gi[TOPK_GROUPS - 1][TOPK_LANES];
  const int row = blockIdx.x;
  const int t = threadIdx.x % TOPK_THREADS, grp = threadIdx.x / TOPK_THREADS;
  const uint16_t* x = L + (int64_t)row * ld;
  float best[TOPK_PER_THREAD];
  int bidx[TOPK_PER_THREAD];
#pragma unroll
  for (int e = 0; e < TOPK_PER_THREAD; ++e) {
    best[e] = -INFINITY;
    bidx[e] = 0;
  }
  const int lane0 = TOPK_PER_THREAD * t;
  const int nsteps = (V + TOPK_LANES - 1) / TOPK_LANES;
  // one lane's update with the value at column c (strictly larger replaces)
  auto take = [&](int e, float v, int c) {
    if (v > best[e]) {
      best[e] = v;
      bidx[e] = c;
    }
  };
  if (vec) {
    // Aligned rows: up to TOPK_UNROLL of this group's steps are requested at
    // once (a row of the Qwen3 vocabulary, 75 steps, in one round), then
    // used in column order.  A step past the row, or the partial last step,
    // reads nothing here and is handled below.
    const int full = V / TOPK_LANES;   // steps whose 2048 columns all exist
    for (int s0 = grp; s0 < full; s0 += TOPK_GROUPS * TOPK_UNROLL) {
      u32x4 raw[TOPK_UNROLL];
#pragma unroll
      for (int u = 0; u < TOPK_UNROLL; ++u) {
        const int st = s0 + u * TOPK_GROUPS;
        raw[u] = st < full ? ld16(x + st * TOPK_LANES + lane0) : u32x4{0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u};
      }
#pragma unroll
      for (int u = 0; u < TOPK_UNROLL; ++u) {
        const int c0 = (s0 + u * TOPK_GROUPS) * TOPK_LANES + lane0;   // -inf padding never replaces
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          take(2 * q, bf2f(raw[u][q] & 0xFFFFu), c0 + 2 * q);
          take(2 * q + 1, bf2f(raw[u][q] >> 16), c0 + 2 * q + 1);
        }
      }
    }
    if (full < nsteps && full % TOPK_GROUPS == grp) {   // the partial last step, element by element
      const int c0 = full * TOPK_LANES + lane0;
#pragma unroll
      for (int e = 0; e < TOPK_PER_THREAD; ++e)
        if (c0 + e < V) take(e, bf2f(x[c0 + e]), c0 + e);
    }
  } else {
    for (int st = grp; st < nsteps; st += TOPK_GROUPS) {
      const int c0 = st * TOPK_LANES + lane0;
#pragma unroll
      for (int e = 0; e < TOPK_PER_THREAD; ++e)
        if (c0 + e < V) take(e, bf2f(x[c0 + e]), c0 + e);
    }
  }
  // Merge the groups' lane maxima into group 0: larger value, then the lower
  // column (a lane with no value above -inf keeps column 0 in every group).
  if (grp > 0) {
#pragma unroll
    for (int e = 0; e < TOPK_PER_THREAD; ++e) {
      s_gv[grp - 1][lane0 + e] = best[e];
      s_gi[grp - 1][lane0 + e] = bidx[e];
    }
  }
  __syncthreads();
  if (grp == 0) {
#pragma unroll
    for (int g = 0; g < TOPK_GROUPS - 1; ++g)
#pragma unroll
      for (int e = 0; e < TOPK_PER_THREAD; ++e) {
        const float ov = s_gv[g][lane0 + e];
        const int oi = s_gi[g][lane0 + e];
        if (ov > best[e] || (ov == best[e] && oi < bidx[e])) {
          best[e] = ov;
          bidx[e] = oi;
        }
      }
  }
  // Selection by one wave, without workgroup barriers: the 2048 lane maxima go
  // to LDS, lane l of wave 0 takes lanes l, l + 64, ..., and each round is a
  // wave (max value, min column) reduction followed by removing the chosen
  // column's lane (every entry holding that column: a lane that saw no value
  // above -inf keeps column 0).
  __syncthreads();   // group 0 has read the other groups' maxima
  if (grp == 0) {
#pragma unroll
    for (int e = 0; e < TOPK_PER_THREAD; ++e) {
      s_gv[0][lane0 + e] = best[e];
      s_gi[0][lane0 + e] = bidx[e];
    }
  }
  __syncthreads();
  if (threadIdx.x >= 64) return;   // no barrier follows
  constexpr int PER = TOPK_LANES / 64;
  const int lane = threadIdx.x;
  float bv[PER];
  int bi[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    bv[i] = s_gv[0][lane + 64 * i];
    bi[i] = s_gi[0][lane + 64 * i];
  }
  for (int k = 0; k < K; ++k) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) m = fmaxf(m, bv[i]);
    int ci = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (bv[i] == m && bi[i] < ci) ci = bi[i];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float om = __shfl_xor(m, off);
      const int oi = __shfl_xor(ci, off);
      if (om > m || (om == m && oi < ci)) {
        m = om;
        ci = oi;
      }
    }
    if (lane == 0) {
      vals[(int64_t)row * K + k] = m;
      idxs[(int64_t)row * K + k] = ci;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (bi[i] == ci) bv[i] = -INFINITY;
  }
}

}  // namespace sk

extern "C" int sk_topk_bf16(const sk_bf16* L, int64_t ld, int N, int V, int K, float* vals, int32_t* idxs,
                            hipStream_t stream) {
  if (N < 0 || V < 1 || ld < V || K < 1 || K > sk::TOPK_MAX_K || N > 0x7FFFFFFF) return SK_ERR_SHAPE;
  if (N == 0) return SK_OK;
  if (!L || !vals || !idxs) return SK_ERR_NULL;
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess ||
      strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return SK_ERR_DEVICE;
  const int vec = ((reinterpret_cast<uintptr_t>(L) & 15u) == 0 && (ld & 7) == 0) ? 1 : 0;
  sk::topk_kernel<<<dim3((unsigned)N), dim3(sk::TOPK_THREADS * sk::TOPK_GROUPS), 0, stream>>>(L, ld, V, K, vec, vals, idxs);
  return hipGetLastError() == hipSuccess ? SK_OK : SK_ERR_LAUNCH;
}
