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
// MI355X mapping: one workgroup of 256 threads per row; thread t owns lanes
// 8t .. 8t+7, so one 16-byte load per thread reads 1 KiB contiguous per wave
// (4 KiB per workgroup and sweep step).  The final selection is K rounds of a
// workgroup (max value, min column) reduction through LDS.
#include "starter_amd.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include "sk_kernels.hpp"

namespace sk {

constexpr int TOPK_LANES = 2048;   // the reference's BLOCK
constexpr int TOPK_THREADS = 256;
constexpr int TOPK_PER_THREAD = TOPK_LANES / TOPK_THREADS;   // 8 lanes per thread
constexpr int TOPK_MAX_K = 64;

__global__ void __launch_bounds__(TOPK_THREADS) topk_kernel(const uint16_t* __restrict__ L, int64_t ld, int V,
                                                             int K, int vec, float* __restrict__ vals,
                                                             int32_t* __restrict__ idxs) {
  __shared__ float s_v[TOPK_THREADS / 64];
  __shared__ int s_i[TOPK_THREADS / 64];
  const int row = blockIdx.x, t = threadIdx.x;
  const uint16_t* x = L + (int64_t)row * ld;
  float best[TOPK_PER_THREAD];
  int bidx[TOPK_PER_THREAD];
#pragma unroll
  for (int e = 0; e < TOPK_PER_THREAD; ++e) {
    best[e] = -INFINITY;
    bidx[e] = 0;
  }
  const int lane0 = TOPK_PER_THREAD * t;
  for (int start = 0; start < V; start += TOPK_LANES) {
    const int c0 = start + lane0;
    float v[TOPK_PER_THREAD];
    if (vec && c0 + TOPK_PER_THREAD <= V) {
      const u32x4 w = ld16(x + c0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[2 * q] = bf2f(w[q] & 0xFFFFu);
        v[2 * q + 1] = bf2f(w[q] >> 16);
      }
    } else {
#pragma unroll
      for (int e = 0; e < TOPK_PER_THREAD; ++e) v[e] = c0 + e < V ? bf2f(x[c0 + e]) : -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < TOPK_PER_THREAD; ++e) {
      if (v[e] > best[e]) {   // strict: the first occurrence of a value keeps its lane
        best[e] = v[e];
        bidx[e] = c0 + e;
      }
    }
  }
  const int lane = t & 63, wave = t >> 6;
  for (int k = 0; k < K; ++k) {
    // Thread candidate: max value, lowest column among its lanes holding it.
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < TOPK_PER_THREAD; ++e) m = fmaxf(m, best[e]);
    int ci = 0x7FFFFFFF;
#pragma unroll
    for (int e = 0; e < TOPK_PER_THREAD; ++e)
      if (best[e] == m && bidx[e] < ci) ci = bidx[e];
    // Wave, then workgroup: larger value wins, then the lower column.
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
      s_v[wave] = m;
      s_i[wave] = ci;
    }
    __syncthreads();
    float M = s_v[0];
    int I = s_i[0];
#pragma unroll
    for (int w = 1; w < TOPK_THREADS / 64; ++w)
      if (s_v[w] > M || (s_v[w] == M && s_i[w] < I)) {
        M = s_v[w];
        I = s_i[w];
      }
    __syncthreads();   // s_v / s_i are rewritten by the next round
    if (t == 0) {
      vals[(int64_t)row * K + k] = M;
      idxs[(int64_t)row * K + k] = I;
    }
#pragma unroll
    for (int e = 0; e < TOPK_PER_THREAD; ++e)
      if (bidx[e] == I) best[e] = -INFINITY;
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
  sk::topk_kernel<<<dim3((unsigned)N), dim3(sk::TOPK_THREADS), 0, stream>>>(L, ld, V, K, vec, vals, idxs);
  return hipGetLastError() == hipSuccess ? SK_OK : SK_ERR_LAUNCH;
}
