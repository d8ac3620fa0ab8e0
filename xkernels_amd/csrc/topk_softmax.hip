// The MoE router step: softmax over the expert axis in fp32, top-k selection in
// descending probability with ties broken by ascending expert id, optional
// renormalisation of the selected weights (contract of the reference's
// src/xkernels/ops/moe/topk_softmax.py:33-95 and its Op Spec).
//
// One wave64 owns one row at a time. Lane l holds experts l, l+64, l+128, ...
// (every load instruction of the wave reads one contiguous run of logits), so a
// row of E experts sits in VPT = ceil(E/64) (rounded to a power of two)
// registers per lane. Max and sum are wave reductions; each of the k rounds
// takes the wave-wide largest (probability, -id) key below the previous
// round's winner with one xor-shuffle butterfly.
// Selections are staged in LDS so the renormalisation and the [M, k] output
// writes are contiguous across lanes.
//
// HBM bound: M*E logits in, M*k (weight, id) pairs out; no scratch. Rows of
// more than 2048 experts take a streaming variant (below).
#include <stdint.h>

#include "common.h"

namespace xk {
namespace {

constexpr int kTsWaves = 4;
constexpr int kTsThreads = kTsWaves * 64;

template <typename T>
__device__ __forceinline__ float logit_at(const T* p);
template <>
__device__ __forceinline__ float logit_at<uint16_t>(const uint16_t* p) {  // bf16 bits
  return __uint_as_float(uint32_t(*p) << 16);
}
template <>
__device__ __forceinline__ float logit_at<_Float16>(const _Float16* p) {
  return float(*p);
}
template <>
__device__ __forceinline__ float logit_at<float>(const float* p) {
  return *p;
}

// The reference's stable descending sort (torch.sort, topk_softmax.py:88)
// orders experts by probability, NaN above every number, and equal keys (NaN
// and NaN included) by lower id. One 64-bit key per expert encodes that order
// as an unsigned integer order: the high word is 0xFFFFFFFE for NaN and the
// probability's bit pattern + 1 otherwise (probabilities are +0 .. 1, whose
// bit patterns are ordered like the values; 0 is left for padding), the low
// word ~id (a lower id gives the larger key). Keys are unique and below ~0,
// the bound of the first selection, so selection t takes the largest key
// below selection t-1's. A row with a NaN or +inf logit, or only -inf
// logits, softmaxes to all NaN (as torch's does: the NaN or the inf - inf
// reaches the sum), so it selects experts 0 .. k-1 with NaN weights.
__device__ __forceinline__ uint64_t rank_key(float p, int e) {
  const uint32_t hi = __builtin_isnan(p) ? 0xFFFFFFFEu : __float_as_uint(p) + 1u;
  return (uint64_t(hi) << 32) | uint32_t(~e);
}
__device__ __forceinline__ float key_prob(uint64_t key) {
  const uint32_t hi = uint32_t(key >> 32);
  return hi == 0xFFFFFFFEu ? __builtin_nanf("") : __uint_as_float(hi - 1u);
}
__device__ __forceinline__ int key_id(uint64_t key) { return int(~uint32_t(key)); }

// Largest key of the wave.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t b) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = __shfl_xor(uint32_t(b), off), hi = __shfl_xor(uint32_t(b >> 32), off);
    const uint64_t o = (uint64_t(hi) << 32) | lo;
    b = o > b ? o : b;
  }
  return b;
}

template <typename T, int VPT>
__global__ void __launch_bounds__(kTsThreads)
topk_softmax_rows(const T* __restrict__ logits, int64_t M, int E, int k, int renorm,
                  float* __restrict__ w_out, int32_t* __restrict__ id_out) {
  extern __shared__ __attribute__((aligned(16))) unsigned char ts_lds[];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  float* sel_w = reinterpret_cast<float*>(ts_lds) + wave * 2 * k;
  int32_t* sel_id = reinterpret_cast<int32_t*>(sel_w + k);

  for (int64_t row = int64_t(blockIdx.x) * kTsWaves + wave; row < M;
       row += int64_t(gridDim.x) * kTsWaves) {
    const T* g = logits + row * E;
    float p[VPT];
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int e = j * 64 + lane;
      p[j] = e < E ? logit_at<T>(g + e) : -__builtin_inff();
      mx = fmaxf(mx, p[j]);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int e = j * 64 + lane;
      p[j] = e < E ? expf(p[j] - mx) : 0.f;
      sum += p[j];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    uint64_t key[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int e = j * 64 + lane;
      key[j] = e < E ? rank_key(p[j] / sum, e) : 0;  // padding ranks below every expert
    }

    float picked_sum = 0.f;
    uint64_t prev = ~uint64_t(0);
    for (int t = 0; t < k; ++t) {
      uint64_t best = 0;
#pragma unroll
      for (int j = 0; j < VPT; ++j) best = key[j] < prev && key[j] > best ? key[j] : best;
      // every lane now holds the same winner (k <= E: a real expert)
      prev = wave_max_key(best);
      const float bv = key_prob(prev);
      const int bid = key_id(prev);
      if (lane == 0) {
        sel_w[t] = bv;
        sel_id[t] = bid;
      }
      picked_sum += bv;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int t = lane; t < k; t += 64) {
      const float v = sel_w[t];
      w_out[row * k + t] = renorm ? v / picked_sum : v;
      id_out[row * k + t] = sel_id[t];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Rows of more than 32 * 64 experts: the same selection without holding the
// row in registers. Round t re-reads the row (from L2) and takes the largest
// key below round t-1's winner (the same keys as above): k * E reads and
// exponentials per row. The lane t % 64 writes the t-th selection; the
// renormalisation then rescales each lane's own writes.
template <typename T>
__global__ void __launch_bounds__(kTsThreads)
topk_softmax_rows_stream(const T* __restrict__ logits, int64_t M, int E, int k, int renorm,
                         float* __restrict__ w_out, int32_t* __restrict__ id_out) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  for (int64_t row = int64_t(blockIdx.x) * kTsWaves + wave; row < M;
       row += int64_t(gridDim.x) * kTsWaves) {
    const T* g = logits + row * E;
    float mx = -__builtin_inff();
    for (int e = lane; e < E; e += 64) mx = fmaxf(mx, logit_at<T>(g + e));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float sum = 0.f;
    for (int e = lane; e < E; e += 64) sum += expf(logit_at<T>(g + e) - mx);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    float picked_sum = 0.f;
    uint64_t prev = ~uint64_t(0);
    for (int t = 0; t < k; ++t) {
      uint64_t best = 0;
      for (int e = lane; e < E; e += 64) {
        const uint64_t v = rank_key(expf(logit_at<T>(g + e) - mx) / sum, e);
        best = v < prev && v > best ? v : best;
      }
      prev = wave_max_key(best);
      const float bv = key_prob(prev);
      const int bid = key_id(prev);
      if (lane == (t & 63)) {
        w_out[row * k + t] = bv;
        id_out[row * k + t] = bid;
      }
      picked_sum += bv;
    }
    if (renorm)
      for (int t = lane; t < k; t += 64) w_out[row * k + t] = w_out[row * k + t] / picked_sum;
  }
}

template <typename T, int VPT>
hipError_t launch_vpt(const void* logits, int64_t M, int E, int k, int renorm, float* w,
                      int32_t* ids, hipStream_t stream) {
  const int64_t blocks = (M + kTsWaves - 1) / kTsWaves;
  const int grid = int(blocks < 65536 ? blocks : 65536);
  const size_t lds = size_t(kTsWaves) * 2 * k * sizeof(float);
  hipLaunchKernelGGL((topk_softmax_rows<T, VPT>), dim3(grid), dim3(kTsThreads), lds, stream,
                     static_cast<const T*>(logits), M, E, k, renorm, w, ids);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_typed(const void* logits, int64_t M, int E, int k, int renorm, float* w,
                        int32_t* ids, hipStream_t stream) {
  const int per_lane = (E + 63) / 64;
  if (per_lane <= 1) return launch_vpt<T, 1>(logits, M, E, k, renorm, w, ids, stream);
  if (per_lane <= 2) return launch_vpt<T, 2>(logits, M, E, k, renorm, w, ids, stream);
  if (per_lane <= 4) return launch_vpt<T, 4>(logits, M, E, k, renorm, w, ids, stream);
  if (per_lane <= 8) return launch_vpt<T, 8>(logits, M, E, k, renorm, w, ids, stream);
  if (per_lane <= 16) return launch_vpt<T, 16>(logits, M, E, k, renorm, w, ids, stream);
  if (per_lane <= 32) return launch_vpt<T, 32>(logits, M, E, k, renorm, w, ids, stream);
  const int64_t blocks = (M + kTsWaves - 1) / kTsWaves;
  hipLaunchKernelGGL((topk_softmax_rows_stream<T>), dim3(int(blocks < 65536 ? blocks : 65536)),
                     dim3(kTsThreads), 0, stream, static_cast<const T*>(logits), M, E, k, renorm,
                     w, ids);
  return hipGetLastError();
}

}  // namespace

// Rows beyond 32 * 64 experts take the streaming kernel; ids and indices stay
// 32-bit.
int topk_softmax_max_experts() { return 1 << 30; }

int launch_topk_softmax(const void* logits, int dtype, int64_t M, int64_t E, int64_t k,
                        int renorm, float* w, int32_t* ids, hipStream_t stream) {
  hipError_t e;
  switch (dtype) {
    case XK_DT_BF16:
      e = launch_typed<uint16_t>(logits, M, int(E), int(k), renorm, w, ids, stream);
      break;
    case XK_DT_FP32:
      e = launch_typed<float>(logits, M, int(E), int(k), renorm, w, ids, stream);
      break;
    default:
      e = launch_typed<_Float16>(logits, M, int(E), int(k), renorm, w, ids, stream);
      break;
  }
  if (e != hipSuccess) return set_error(XK_ERR_LAUNCH, "topk_softmax launch: %s", hipGetErrorString(e));
  return XK_OK;
}

}  // namespace xk
