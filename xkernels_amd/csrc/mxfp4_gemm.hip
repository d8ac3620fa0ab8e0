// MXFP4 MoE kernels for gfx950 (the reference's _mxfp4_moe_gemm_kernel,
// src/xkernels/ops/moe/triton/moe_mxfp4_kernel.py:87-352; math of the oracle
// mxfp4_reference.py:28-112 with the dequant of ops/gather/mxfp4.py:39-68).
//
//   stage 0 : gu = bf16(A[m]) @ w13[e]^T (+ b13[e]),  act[t, j] =
//             bf16(silu(min(g, L)) * clamp(u, -L, L)),  g = gu[j], u = gu[ispp + j]
//   stage 1 : slot_out[t, n] = bf16(bf16(act[t] @ w2[e]^T) (+ b2[e, n]))   (fp32 row)
// followed by the weighted top-k combine (reduce.hip). The bf16 roundings sit
// where the reference's bf16 torch ops round (matmul output, bias add, act).
//
// Main path (bf16 activations, hidden and ispp multiples of 128, E <= 512):
// both projections run mxfp4_stream_rs (int4_stream.hip) into fp32 partial
// planes; mxfp4_swiglu_planes below finishes stage 0 and the combine applies
// stage 1's roundings and bias. Every other shape runs mxfp4_stream_gemm: a
// workgroup owns (expert e, a column block) and all of e's routed slots, 32 at
// a time; lane (c, q) of a wave reads 16 bytes = one 32-element e8m0 group of
// its weight row and dequantises it with four v_cvt_scalef32_pk_bf16_fp4 (two
// e2m1 -> two bf16, times 2^(e-127), exact); a 32-row x 256-k activation chunk
// is staged in LDS.
#include <algorithm>
#include <type_traits>

#include "int4_common.h"

namespace xk {
namespace {

constexpr int kChunkGroups = 8;           // 256 k per staged chunk
constexpr int kChunkK = kChunkGroups * 32;
constexpr int kRows = 32;                 // slots per pass (two MFMA row tiles)
constexpr int kStride = kChunkK + 8;      // bf16 elements per LDS row

// Stages one 32 x 256 activation chunk into LDS (bf16). Row r of the pass reads
// source row src_row[r] (< 0: zero row); TA is the activation storage type.
template <typename TA>
__device__ __forceinline__ void load_rows(const TA* src, int64_t ld, int src_row, int g, int G,
                                          uint32_t* areg) {
  if (src_row >= 0 && g < G) {
    const TA* p = src + static_cast<int64_t>(src_row) * ld + g * 32;
    if constexpr (sizeof(TA) == 2) {
      const u32x4* v = reinterpret_cast<const u32x4*>(p);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4 x = v[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) areg[4 * j + i] = x[i];
      }
    } else {
      const f32x4* v = reinterpret_cast<const f32x4*>(p);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const f32x4 x = v[j];
        areg[2 * j] = f32_to_bf16(x[0]) | (static_cast<uint32_t>(f32_to_bf16(x[1])) << 16);
        areg[2 * j + 1] = f32_to_bf16(x[2]) | (static_cast<uint32_t>(f32_to_bf16(x[3])) << 16);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) areg[i] = 0u;
  }
}

struct Mxfp4Args {
  const void* A;           // stage 0: [M, hidden] (TA); stage 1: act [numel, ispp] bf16
  const uint8_t* w;        // stage 0: w13 [E, 2*ispp, hidden/2]; stage 1: w2 [E, hidden, ispp/2]
  const uint8_t* ws;       // matching e8m0 scales
  const uint16_t* bias;    // stage 0: b13 [E, 2*ispp]; stage 1: b2 [E, hidden]; nullable
  const int32_t* sorted_ids;
  const int32_t* offsets;
  uint16_t* act;           // stage 0 output [numel, ispp]
  float* slot_out;         // stage 1 output [numel, hidden]
  int K;                   // contraction length (hidden | ispp)
  int rows;                // weight rows per expert (2*ispp | hidden)
  int ncols;               // output columns (ispp | hidden)
  int numel, top_k;
  float limit;             // swiglu clamp, <= 0 disables
};

// STAGE 0: each wave owns 16 act columns j and reads gate row j and up row
// ispp + j; the workgroup covers 64 columns. STAGE 1: each wave owns two 16-col
// tiles of hidden; the workgroup covers 128 columns.
template <int STAGE, typename TA>
__global__ void __launch_bounds__(256)
mxfp4_stream_gemm(Mxfp4Args p) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[kRows * kStride];
  __shared__ int slot_lds[kRows];
  __shared__ int src_lds[kRows];

  const int e = blockIdx.y;
  const int beg = p.offsets[e], end = p.offsets[e + 1];
  if (beg >= end) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, q = lane >> 4;
  const int K = p.K, G = K >> 5, KB = K >> 1;  // bytes per weight row
  constexpr int kColsPerWave = STAGE == 0 ? 16 : 32;
  const int col_base = blockIdx.x * (4 * kColsPerWave) + wave * kColsPerWave;

  // weight rows of the two column tiles
  const uint8_t* wrow[2];
  const uint8_t* srow[2];
  int col[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    int row;
    if (STAGE == 0) {
      col[c] = col_base + c16;                             // act column j
      row = min(col[c], p.ncols - 1) + (c ? p.ncols : 0);  // gate row j, up row ispp + j
    } else {
      col[c] = col_base + 16 * c + c16;
      row = min(col[c], p.ncols - 1);
    }
    wrow[c] = p.w + (static_cast<int64_t>(e) * p.rows + row) * KB;
    srow[c] = p.ws + (static_cast<int64_t>(e) * p.rows + row) * G;
  }
  const int st_r = tid >> 3, st_g = tid & 7;

  for (int pass = beg; pass < end; pass += kRows) {
    const int ntiles = min(2, (end - pass) >> 4);
    __syncthreads();
    if (tid < kRows) {
      int slot = -1, src = -1;
      if (tid < ntiles * 16) {
        const int s = p.sorted_ids[pass + tid];
        if (s < p.numel) { slot = s; src = STAGE == 0 ? s / p.top_k : s; }
      }
      slot_lds[tid] = slot;
      src_lds[tid] = src;
    }
    __syncthreads();
    const int my_src = src_lds[st_r];

    f32x4 acc[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint32_t areg[16];
    u32x4 wcur[2][2], wnext[2][2];  // [col tile][half of the chunk]
    float scur[2][2], snext[2][2];
    auto load_w = [&](int g0, u32x4 (*wr)[2], float (*sr)[2]) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int g = g0 + 4 * h + q;
          if (g < G) {
            const uint32_t b = srow[c][g];
            wr[c][h] = b == 0xFFu ? u32x4{0u, 0u, 0u, 0u}
                                  : *reinterpret_cast<const u32x4*>(wrow[c] + g * 16);
            sr[c][h] = e8m0_scale(b);
          } else {
            wr[c][h] = u32x4{0u, 0u, 0u, 0u};
            sr[c][h] = 0.f;
          }
        }
    };
    const TA* asrc = static_cast<const TA*>(p.A);
    load_rows<TA>(asrc, K, my_src, st_g, G, areg);
    load_w(0, wcur, scur);

    for (int g0 = 0; g0 < G; g0 += kChunkGroups) {
      __syncthreads();
      {
        u32x4* dst = reinterpret_cast<u32x4*>(a_lds + st_r * kStride + st_g * 32);
#pragma unroll
        for (int s = 0; s < 4; ++s)
          dst[s] = u32x4{areg[4 * s], areg[4 * s + 1], areg[4 * s + 2], areg[4 * s + 3]};
      }
      __syncthreads();
      const int gn = g0 + kChunkGroups;
      if (gn < G) {
        load_rows<TA>(asrc, K, my_src, gn + st_g, G, areg);
        load_w(gn, wnext, snext);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (g0 + 4 * h >= G) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bf16x8 bfrag[2];
#pragma unroll
          for (int c = 0; c < 2; ++c) bfrag[c] = fp4x8_to_bf16(wcur[c][h][j], scur[c][h]);
          // A columns matching lane q's weights: group g0 + 4h + q, elements 8j..8j+7
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            if (t >= ntiles) break;
            const bf16x8 afrag = *reinterpret_cast<const bf16x8*>(
                a_lds + (t * 16 + c16) * kStride + (4 * h + q) * 32 + 8 * j);
#pragma unroll
            for (int c = 0; c < 2; ++c)
              acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, bfrag[c], acc[t][c], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h) { wcur[c][h] = wnext[c][h]; scur[c][h] = snext[c][h]; }
    }

#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t >= ntiles) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int slot = slot_lds[t * 16 + q * 4 + i];
        if (slot < 0) continue;
        if (STAGE == 0) {
          const int j = col[0];
          if (j >= p.ncols) continue;
          const uint16_t* b = p.bias ? p.bias + static_cast<int64_t>(e) * 2 * p.ncols : nullptr;
          p.act[static_cast<int64_t>(slot) * p.ncols + j] =
              mxfp4_swiglu(acc[t][0][i], acc[t][1][i], b, j, p.ncols, p.limit);
        } else {
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int n = col[c];
            if (n >= p.ncols) continue;
            float d = round_bf16(acc[t][c][i]);
            if (p.bias != nullptr)
              d = round_bf16(d + bf16_to_f32(p.bias[static_cast<int64_t>(e) * p.ncols + n]));
            p.slot_out[static_cast<int64_t>(slot) * p.ncols + n] = d;
          }
        }
      }
    }
  }
}

// Gate/up epilogue for the stream path: the projection's S fp32 partial planes
// [S, numel, 2 ispp] are summed and finished exactly like the per-workgroup
// epilogue above: gu = bf16(sum) (+ b13 -> bf16), g clamped from above, u on
// both sides, act = bf16(silu(g) * u). Four columns per thread; slots whose
// expert is not local (never computed) are skipped.
__global__ void __launch_bounds__(256)
mxfp4_swiglu_planes(const float* __restrict__ planes, int S, int64_t numel, int ispp,
                    const uint16_t* __restrict__ b13, const int32_t* __restrict__ topk_ids,
                    const int32_t* __restrict__ emap, int num_global, int num_local, float limit,
                    uint16_t* __restrict__ act) {
  const int64_t per_row = ispp / 4;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= numel * per_row) return;
  const int64_t t = idx / per_row;
  const int j0 = static_cast<int>(idx - t * per_row) * 4;
  const int e = map_expert(topk_ids[t], emap, num_global, num_local);
  if (e < 0) return;
  const int64_t pstride = numel * 2 * ispp;
  const float* row = planes + t * 2 * ispp;
  // the planes in groups of four loads in flight (a decode batch of one token
  // has 16 K slices: 9.5 -> 6.8 us; groups of eight measured 12.2 us)
  f32x4 g = *reinterpret_cast<const f32x4*>(row + j0);
  f32x4 u = *reinterpret_cast<const f32x4*>(row + ispp + j0);
  int sl = 1;
  for (; sl + 3 < S; sl += 4) {
    f32x4 gs[4], us[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      gs[i] = *reinterpret_cast<const f32x4*>(row + (sl + i) * pstride + j0);
      us[i] = *reinterpret_cast<const f32x4*>(row + (sl + i) * pstride + ispp + j0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      g += gs[i];
      u += us[i];
    }
  }
  for (; sl < S; ++sl) {
    g += *reinterpret_cast<const f32x4*>(row + sl * pstride + j0);
    u += *reinterpret_cast<const f32x4*>(row + sl * pstride + ispp + j0);
  }
  uint16_t r[4];
  const uint16_t* b = b13 ? b13 + static_cast<int64_t>(e) * 2 * ispp : nullptr;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = mxfp4_swiglu(g[i], u[i], b, j0 + i, ispp, limit);
  uint2 o;
  o.x = r[0] | (static_cast<uint32_t>(r[1]) << 16);
  o.y = r[2] | (static_cast<uint32_t>(r[3]) << 16);
  *reinterpret_cast<uint2*>(act + t * ispp + j0) = o;
}

}  // namespace

int device_cu_count();

int mxfp4_block_size() { return 16; }

int launch_mxfp4_stage(int stage, const void* A, int a_dtype, const uint8_t* w,
                       const uint8_t* ws, const uint16_t* bias, int64_t E, int64_t K,
                       int64_t rows, int64_t ncols, const int32_t* sorted_ids,
                       const int32_t* offsets, int64_t numel, int64_t top_k, float limit,
                       uint16_t* act, float* slot_out, hipStream_t stream) {
  XK_REQUIRE(K % 32 == 0 && K >= 32, "mxfp4: contraction %lld not a multiple of 32",
             (long long)K);
  XK_REQUIRE(reinterpret_cast<uintptr_t>(A) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0,
             "mxfp4: activations and weights must be 16-byte aligned");
  if (numel == 0) return XK_OK;
  Mxfp4Args a{A, w, ws, bias, sorted_ids, offsets, act, slot_out, int(K), int(rows),
              int(ncols), int(numel), int(top_k), limit};
  if (stage == 0) {
    const dim3 grid(static_cast<unsigned>(cdiv(ncols, 64)), static_cast<unsigned>(E));
    if (a_dtype == XK_DT_BF16)
      hipLaunchKernelGGL((mxfp4_stream_gemm<0, uint16_t>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((mxfp4_stream_gemm<0, float>), grid, dim3(256), 0, stream, a);
    XK_CHECK_LAUNCH("mxfp4_stream_gemm<0>");
  } else {
    const dim3 grid(static_cast<unsigned>(cdiv(ncols, 128)), static_cast<unsigned>(E));
    hipLaunchKernelGGL((mxfp4_stream_gemm<1, uint16_t>), grid, dim3(256), 0, stream, a);
    XK_CHECK_LAUNCH("mxfp4_stream_gemm<1>");
  }
  return XK_OK;
}

}  // namespace xk

namespace xk {

int launch_mxfp4_swiglu(const float* planes, int S, int64_t numel, int64_t ispp, const uint16_t* b13,
                        const int32_t* topk_ids, const int32_t* emap, int num_global, int num_local,
                        float limit, uint16_t* act, hipStream_t stream) {
  XK_REQUIRE(ispp % 4 == 0, "mxfp4 swiglu: ispp %lld not a multiple of 4", (long long)ispp);
  const int64_t n = numel * (ispp / 4);
  if (n == 0) return XK_OK;
  hipLaunchKernelGGL(mxfp4_swiglu_planes, dim3(static_cast<unsigned>(cdiv(n, 256))), dim3(256), 0,
                     stream, planes, S, numel, int(ispp), b13, topk_ids, emap, num_global, num_local,
                     limit, act);
  XK_CHECK_LAUNCH("mxfp4_swiglu_planes");
  return XK_OK;
}

}  // namespace xk
