// Weighted top-k reduction kernels for gfx950.
//
//   moe_sum_reduce  (sum_reduce.py:20-39):
//     out[m, h] = s * sum_k w[m, k] * y[m, k, h]        fp32 accumulate, y dtype out
//   top-k combine   (the reduce after the grouped GEMMs; reference.py:59-70,
//                    mxfp4_reference.py:104-112):
//     out[m, n] = sum_j valid(m, j) * [w[m, j]] * slot_out[m*top_k + j, n]
//
// Pure HBM streaming. One thread owns VEC consecutive elements of one output
// row and walks the top_k inputs with 16-byte loads (bf16: 8 elements, fp32:
// 2 x 4), so every load instruction of a wavefront covers 1 KiB contiguous.
// The k loop is fully unrolled for the common top_k so all loads issue before
// the first add.
#include <type_traits>

#include "common.h"

namespace xk {
namespace {

template <typename T, int VEC> struct vec_io;
// bf16 inputs (moe_sum_reduce) are read exactly once: non-temporal loads keep
// them from displacing useful cache lines (measured 192 -> 178 us on the
// [8192, 8, 7168] bf16 sum). The fp32 inputs (the grouped GEMMs' partial rows,
// written just before) are read with the default policy: C2 step 174.2 ->
// 172.4 us, C4 call 136.0 -> 134.2 us.
template <> struct vec_io<uint16_t, 8> {
  __device__ __forceinline__ static void load(const uint16_t* p, float* v) {
    const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(r[i] << 16);
      v[2 * i + 1] = __uint_as_float(r[i] & 0xFFFF0000u);
    }
  }
  __device__ __forceinline__ static void store(uint16_t* p, const float* v) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      r[i] = static_cast<uint32_t>(f32_to_bf16(v[2 * i])) |
             (static_cast<uint32_t>(f32_to_bf16(v[2 * i + 1])) << 16);
    *reinterpret_cast<u32x4*>(p) = r;
  }
};
template <> struct vec_io<float, 8> {
  __device__ __forceinline__ static void load(const float* p, float* v) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *(reinterpret_cast<const f32x4*>(p) + 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
  }
  __device__ __forceinline__ static void store(float* p, const float* v) {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) { a[i] = v[i]; b[i] = v[4 + i]; }
    reinterpret_cast<f32x4*>(p)[0] = a;
    reinterpret_cast<f32x4*>(p)[1] = b;
  }
};
template <> struct vec_io<float, 4> {
  __device__ __forceinline__ static void load(const float* p, float* v) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = a[i];
  }
  __device__ __forceinline__ static void store(float* p, const float* v) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  }
};
template <> struct vec_io<uint16_t, 4> {
  __device__ __forceinline__ static void store(uint16_t* p, const float* v) {
    uint2 r;
    r.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
    r.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
    *reinterpret_cast<uint2*>(p) = r;
  }
};
template <typename T> struct vec_io<T, 1> {
  __device__ __forceinline__ static void load(const T* p, float* v) { v[0] = io<T>::load(p); }
  __device__ __forceinline__ static void store(T* p, const float* v) { io<T>::store(p, v[0]); }
};

// Row weights: per (m, k) multiplier applied to y[m, k, :]. Covers the plain
// sum (no weights), weights in fp32 or bf16, and the combine's validity mask.
struct RowWeights {
  const void* w;        // [M, top_k] or null
  int w_dtype;          // XK_DT_*
  const int32_t* ids;   // [M, top_k] or null (no mask)
  const int32_t* emap;  // nullable
  int num_global, num_local;
  // MXFP4 down projection finished here: a slot's summed row is rounded to
  // bf16, then bias[expert] is added and the sum rounded to bf16 again
  // (the reference's bf16 matmul output and bias add)
  const uint16_t* post_bias = nullptr;  // [num_local, H] bf16 or null
  int post_round = 0;

  __device__ __forceinline__ float get(int64_t idx) const {
    if (w == nullptr) return 1.0f;
    return (w_dtype == XK_DT_FP32) ? static_cast<const float*>(w)[idx]
                                   : bf16_to_f32(static_cast<const uint16_t*>(w)[idx]);
  }
  // Dropped slots are skipped (their rows were never written, so they are
  // selected away rather than multiplied by zero).
  __device__ __forceinline__ bool valid(int64_t idx) const {
    return ids == nullptr || map_expert(ids[idx], emap, num_global, num_local) >= 0;
  }
  template <int VEC>
  __device__ __forceinline__ void post(int64_t idx, int64_t H, int64_t h, float* v) const {
    if (!post_round) return;
    const int e = ids == nullptr ? -1 : map_expert(ids[idx], emap, num_global, num_local);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      v[i] = round_bf16(v[i]);
      if (post_bias != nullptr && e >= 0)
        v[i] = round_bf16(v[i] + bf16_to_f32(post_bias[static_cast<int64_t>(e) * H + h + i]));
    }
  }
};

// y may hold `nparts` planes (partial sums over K) `pstride` elements apart;
// they are added before weighting.
template <typename Tin, typename Tout, int VEC, int KFIX>
__global__ void __launch_bounds__(256)
topk_reduce(const Tin* __restrict__ y, int64_t M, int top_k_rt, int64_t H, RowWeights rw,
            float scale, Tout* __restrict__ out, int nparts, int64_t pstride) {
  const int top_k = KFIX > 0 ? KFIX : top_k_rt;
  const int64_t chunks_per_row = H / VEC;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= M * chunks_per_row) return;
  const int64_t m = idx / chunks_per_row;
  const int64_t h = (idx - m * chunks_per_row) * VEC;
  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.0f;
  const Tin* src = y + (m * top_k) * H + h;
  if (KFIX > 0) {
    float v[KFIX > 0 ? KFIX : 1][VEC];
    float wk[KFIX > 0 ? KFIX : 1];
    bool ok[KFIX > 0 ? KFIX : 1];
#pragma unroll
    for (int k = 0; k < KFIX; ++k) {
      wk[k] = rw.get(m * top_k + k);
      ok[k] = rw.valid(m * top_k + k);
      vec_io<Tin, VEC>::load(src + k * H, v[k]);
    }
    for (int p = 1; p < nparts; ++p) {
#pragma unroll
      for (int k = 0; k < KFIX; ++k) {
        float t[VEC];
        vec_io<Tin, VEC>::load(src + p * pstride + k * H, t);
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[k][i] += t[i];
      }
    }
#pragma unroll
    for (int k = 0; k < KFIX; ++k) {
      rw.template post<VEC>(m * top_k + k, H, h, v[k]);
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[i] += ok[k] ? v[k][i] * wk[k] : 0.0f;
    }
  } else {
    for (int k = 0; k < top_k; ++k) {
      if (!rw.valid(m * top_k + k)) continue;
      float v[VEC];
      const float wk = rw.get(m * top_k + k);
      vec_io<Tin, VEC>::load(src + k * H, v);
      for (int p = 1; p < nparts; ++p) {
        float t[VEC];
        vec_io<Tin, VEC>::load(src + p * pstride + k * H, t);
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[i] += t[i];
      }
      rw.template post<VEC>(m * top_k + k, H, h, v);
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[i] += v[i] * wk;
    }
  }
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] *= scale;
  vec_io<Tout, VEC>::store(out + m * H + h, acc);
}

template <typename Tin, typename Tout, int VEC>
int launch_vec(const Tin* y, int64_t M, int top_k, int64_t H, const RowWeights& rw,
               float scale, Tout* out, int nparts, int64_t pstride, hipStream_t stream) {
  const int64_t n = M * (H / VEC);
  if (n == 0) return XK_OK;
  const dim3 grid(static_cast<unsigned>(cdiv(n, 256))), block(256);
  switch (top_k) {
#define XK_K(K)                                                                      \
  case K:                                                                            \
    hipLaunchKernelGGL((topk_reduce<Tin, Tout, VEC, K>), grid, block, 0, stream, y, M, \
                       top_k, H, rw, scale, out, nparts, pstride);                   \
    break;
    XK_K(1) XK_K(2) XK_K(4) XK_K(6) XK_K(8)
#undef XK_K
    default:
      hipLaunchKernelGGL((topk_reduce<Tin, Tout, VEC, 0>), grid, block, 0, stream, y, M,
                         top_k, H, rw, scale, out, nparts, pstride);
  }
  XK_CHECK_LAUNCH("topk_reduce");
  return XK_OK;
}

template <typename Tin, typename Tout>
int launch_reduce(const Tin* y, int64_t M, int top_k, int64_t H, const RowWeights& rw,
                  float scale, Tout* out, hipStream_t stream, int nparts = 1,
                  int64_t pstride = 0) {
  const bool aligned = (reinterpret_cast<uintptr_t>(y) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(out) % 16 == 0) && (pstride % 8 == 0);
  // fp32 inputs (the combine's per-slot rows) take 4 outputs per thread below
  // 2^22 outputs: a decode batch (M = 64, N = 4096) then spans every CU
  // (measured 8.1 -> 6.2 us on the C2 combine); larger ones take 8 (the C5
  // combine, 4096 x 4096: 111.9 -> 103.5 us). bf16 inputs keep one 16-byte
  // load per slot.
  if constexpr (std::is_same<Tin, float>::value) {
    if (H % 4 == 0 && aligned && !(H % 8 == 0 && M * H >= (int64_t(1) << 22)))
      return launch_vec<Tin, Tout, 4>(y, M, top_k, H, rw, scale, out, nparts, pstride, stream);
  }
  if (H % 8 == 0 && aligned)
    return launch_vec<Tin, Tout, 8>(y, M, top_k, H, rw, scale, out, nparts, pstride, stream);
  return launch_vec<Tin, Tout, 1>(y, M, top_k, H, rw, scale, out, nparts, pstride, stream);
}

}  // namespace

int launch_sum_reduce(const void* y, int y_dtype, int64_t M, int64_t top_k, int64_t H,
                      const void* w, int w_dtype, float scale, void* out,
                      hipStream_t stream) {
  XK_REQUIRE(y_dtype == XK_DT_BF16 || y_dtype == XK_DT_FP32, "sum_reduce: bad y dtype %d", y_dtype);
  XK_REQUIRE(w == nullptr || w_dtype == XK_DT_BF16 || w_dtype == XK_DT_FP32,
             "sum_reduce: bad w dtype %d", w_dtype);
  XK_REQUIRE(M >= 0 && top_k >= 0 && H >= 0, "sum_reduce: negative size");
  XK_REQUIRE(top_k <= 1024, "sum_reduce: top_k=%lld > 1024", (long long)top_k);
  XK_REQUIRE(M * H == 0 || (y && out), "sum_reduce: null pointer");
  const RowWeights rw{w, w_dtype, nullptr, nullptr, 0, 0};
  if (y_dtype == XK_DT_BF16)
    return launch_reduce(static_cast<const uint16_t*>(y), M, int(top_k), H, rw, scale,
                         static_cast<uint16_t*>(out), stream);
  return launch_reduce(static_cast<const float*>(y), M, int(top_k), H, rw, scale,
                       static_cast<float*>(out), stream);
}

int launch_topk_combine(const float* slot_out, int64_t M, int64_t top_k, int64_t N,
                        const float* topk_w, int mul_routed_weight, const int32_t* topk_ids,
                        int num_local, const int32_t* emap, int num_global, void* out,
                        int out_dtype, int nparts, hipStream_t stream, const uint16_t* post_bias,
                        int post_round) {
  XK_REQUIRE(nparts >= 1 && nparts <= 64, "combine: nparts=%d outside [1, 64]", nparts);
  XK_REQUIRE(out_dtype == XK_DT_BF16 || out_dtype == XK_DT_FP32, "combine: bad out dtype %d",
             out_dtype);
  XK_REQUIRE(!mul_routed_weight || topk_w, "combine: null topk_w");
  XK_REQUIRE(top_k >= 1 && top_k <= 1024, "combine: top_k=%lld outside [1, 1024]",
             (long long)top_k);
  const RowWeights rw{mul_routed_weight ? topk_w : nullptr, XK_DT_FP32, topk_ids, emap,
                      num_global, num_local, post_bias, post_round};
  const int64_t pstride = M * top_k * N;
  if (out_dtype == XK_DT_BF16)
    return launch_reduce(slot_out, M, int(top_k), N, rw, 1.0f, static_cast<uint16_t*>(out),
                         stream, nparts, pstride);
  return launch_reduce(slot_out, M, int(top_k), N, rw, 1.0f, static_cast<float*>(out), stream,
                       nparts, pstride);
}

}  // namespace xk
