// Grouped INT4 W4A16 MoE GEMM for gfx950: kernel choice and launch (the
// reference's _fused_moe_int4_kernel launch, src/xkernels/ops/moe/triton/
// moe_int4_kernel.py:291-415; math of the oracle reference.py:22-70 with the
// dequant of w4a16.py:21-50).
//
// For every routed slot t (token m = t / top_k, local expert e) the kernels
// write the un-weighted fp32 row   slot_out[t, n] = sum_k A[m, k] * W[e, n, k]
// with W[e, n, k] = bf16((nibble(e, n, k) - 8) * scale[e, n, k / 32]) for bf16
// activations (the reference rounds the dequantised weight to A's dtype). The
// weighted top-k combine runs afterwards (reduce.hip). Kernels:
//   * int4_stream_rne (int4_stream.hip): decode regime, bf16 A, group 32 —
//     weight streaming with the exact bf16 dequant, K-slice partial planes;
//   * int4_prefill_tile (int4_prefill.hip): prefill regime (>= 17 routed rows
//     per expert on average), MFMA tiles, the same exact dequant;
//   * int4_simple_gemm (below): any dtype, group size or shape the MFMA
//     kernels do not take — one thread per (slot, column), exact dequant
//     rounded to A's dtype like the reference.
#include <algorithm>
#include <type_traits>

#include "int4_common.h"
#include "int4_flags.h"

namespace xk {
namespace {

// One thread per (slot, column); exact dequant rounded to A's dtype.
template <typename TA>
__global__ void __launch_bounds__(256)
int4_simple_gemm(const TA* __restrict__ A, int K, const uint32_t* __restrict__ packed,
                 const uint16_t* __restrict__ scale, int N, int group_size,
                 const int32_t* __restrict__ ids, const int32_t* __restrict__ emap,
                 int num_global, int num_local, int numel, int top_k,
                 float* __restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(numel) * N) return;
  const int t = static_cast<int>(idx / N), n = static_cast<int>(idx - static_cast<int64_t>(t) * N);
  const int e = map_expert(ids[t], emap, num_global, num_local);
  if (e < 0) return;
  const int m = t / top_k;
  const int G = K / group_size;
  const uint32_t* wr = packed + (static_cast<int64_t>(e) * N + n) * (K >> 3);
  const uint16_t* sr = scale + (static_cast<int64_t>(e) * N + n) * G;
  const TA* ar = A + static_cast<int64_t>(m) * K;
  float acc = 0.f;
  for (int kw = 0; kw < (K >> 3); ++kw) {
    const uint32_t w = wr[kw];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = kw * 8 + j;
      const float s = bf16_to_f32(sr[k / group_size]);
      float v = static_cast<float>(static_cast<int>((w >> (4 * j)) & 0xFu) - 8) * s;
      if (sizeof(TA) == 2) v = round_bf16(v);
      acc = fmaf(io<TA>::load(ar + k), v, acc);
    }
  }
  out[static_cast<int64_t>(t) * N + n] = acc;
}

}  // namespace

// Number of compute units of the current device (cached per device).
int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Token-slot block size the MFMA kernels consume (one MFMA row tile).
int int4_block_size() { return 16; }

bool int4_rs_group_ok(int64_t K, int group_size);

// The MFMA kernels take quantisation groups of 32, 64 or 128 and K a multiple
// of 32; bf16 or fp32 activations (fp32: the weight-streaming kernel only).
bool int4_use_stream(int a_dtype, int group_size, int64_t K) {
  return (a_dtype == XK_DT_BF16 || a_dtype == XK_DT_FP32) && K % 32 == 0 &&
         int4_rs_group_ok(K, group_size);
}

bool int4_prefill_ok(int a_dtype, int group_size, int64_t M, int64_t K, int64_t N, int64_t E);
bool int4_rs_ok(int64_t M, int64_t top_k, int64_t K, int64_t N, int64_t E, bool f32a,
                int group_size);
int int4_rs_slices(int64_t K, int64_t N, int64_t numel, int64_t E, bool f32a);
bool int4_rs_self_route_ok(int64_t numel);
int launch_int4_rs(const void* A, bool f32a, int64_t M, int64_t K, const int32_t* packed,
                   const uint16_t* scale, int64_t E, int64_t N, int64_t numel, int64_t top_k,
                   int group_size, const int32_t* sorted_ids, const int32_t* offsets,
                   const int32_t* topk_ids, const int32_t* emap, int num_global, float* slot_out,
                   hipStream_t stream);
int launch_int4_prefill(const void* A, int64_t K, const int32_t* packed, const uint16_t* scale,
                        int64_t E, int64_t N, int64_t numel, int64_t top_k, int group_size,
                        const int32_t* sorted_ids, const int32_t* offsets, float* slot_out,
                        int* queue, hipStream_t stream);

// Routed rows per expert (on average) from which the tile kernel replaces the
// weight-streaming kernel, which streams every expert's weights once per
// 16-row pass. Measured at E = 48, N = 4096, K = 7168, top_k = 8 (uniform
// routing): stream vs tile 177.2 vs 248.4 us at 13.3 rows per expert, 228.9
// vs 248.1 us at 16, 264.4 vs 249.8 us at 18.7, 294.6 vs 249.2 us at 21.3.
constexpr int64_t kPrefillRowsPerExpert = 17;

// The INT4 kernels need no workspace; the argument and this size stay in the
// interface (0 bytes, NULL accepted).
int64_t int4_prefill_queue_bytes();

// The tile kernel's queue; the other kernels need none.
int64_t int4_gemm_workspace_bytes(int64_t M, int64_t K) {
  (void)M;
  (void)K;
  return int4_prefill_queue_bytes();
}

// The grouped-GEMM kernel a call runs, from its shapes and flags only (not
// from pointers), so that the number of partial planes is known before the
// call. Pointer alignment the chosen kernel needs is checked at launch.
enum class Int4Kernel { kSimple, kRs, kTile };

// ep_global > E: the call runs E local experts of ep_global under an expert
// map; the routed rows per local expert are then estimated as those of the
// dense call (numel * E / ep_global slots expected on the local experts), so
// that an expert-parallel rank picks the kernel the dense call picks for the
// same rows per expert. 0: every slot counts against the E experts.
Int4Kernel int4_choose(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K, int a_dtype,
                       int group_size, int flags, int64_t ep_global) {
  if (!int4_use_stream(a_dtype, group_size, K)) return Int4Kernel::kSimple;
  const int64_t numel = M * top_k;
  const int64_t local = ep_global > E ? (numel * E + ep_global - 1) / ep_global : numel;
  const bool f32a = a_dtype == XK_DT_FP32;
  const bool tile_ok = !f32a && int4_prefill_ok(a_dtype, group_size, M, K, N, E);
  const bool rs_ok = int4_rs_ok(M, top_k, K, N, E, f32a, group_size);
  bool tile = tile_ok && local >= kPrefillRowsPerExpert * E;
  if (flags & XK_INT4_TEST_FORCE_TILE) tile = tile_ok;
  if (flags & XK_INT4_TEST_FORCE_STREAM) tile = tile && !rs_ok;
  if (tile) return Int4Kernel::kTile;
  if (rs_ok) return Int4Kernel::kRs;
  return tile_ok ? Int4Kernel::kTile : Int4Kernel::kSimple;
}

// The kernel a call runs, for the C ABI's query: 0 the scalar kernel, 1 the
// decode stream kernel, 2 the prefill tile kernel.
int int4_kernel_code(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K, int a_dtype,
                     int group_size, int flags, int64_t ep_global) {
  switch (int4_choose(M, top_k, E, N, K, a_dtype, group_size, flags, ep_global)) {
    case Int4Kernel::kRs: return 1;
    case Int4Kernel::kTile: return 2;
    default: return 0;
  }
}

// Number of fp32 partial planes [parts, M * top_k, N] the grouped GEMM
// writes: the K slices of the decode stream kernel, else one.
int int4_gemm_parts(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K, int a_dtype,
                    int group_size, int flags, int64_t ep_global) {
  return int4_choose(M, top_k, E, N, K, a_dtype, group_size, flags, ep_global) == Int4Kernel::kRs
             ? int4_rs_slices(K, N, M * top_k, E, a_dtype == XK_DT_FP32)
             : 1;
}

// True when launch_int4_gemm may be called without align outputs (the decode
// kernel then routes the slots itself).
bool int4_gemm_self_routes(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K, int a_dtype,
                           int group_size, int flags, int64_t ep_global) {
  return int4_choose(M, top_k, E, N, K, a_dtype, group_size, flags, ep_global) == Int4Kernel::kRs &&
         int4_rs_self_route_ok(M * top_k);
}

int launch_int4_gemm(const void* A, int a_dtype, int64_t M, int64_t K, const int32_t* packed,
                     const uint16_t* scale, int64_t E, int64_t N, int group_size,
                     const int32_t* topk_ids, int64_t top_k, const int32_t* emap,
                     int num_global, const int32_t* sorted_ids, const int32_t* offsets,
                     float* slot_out, int flags, int64_t ep_global, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream) {
  XK_REQUIRE(a_dtype == XK_DT_BF16 || a_dtype == XK_DT_FP32, "int4: bad A dtype %d", a_dtype);
  XK_REQUIRE((flags & ~(XK_INT4_TEST_FORCE_TILE | XK_INT4_TEST_FORCE_STREAM)) == 0,
             "int4: unknown flags 0x%x (pass 0)", flags);
  XK_REQUIRE(M >= 0 && top_k >= 1 && E >= 1 && N >= 1 && K >= 8, "int4: bad sizes");
  XK_REQUIRE(K % 8 == 0, "int4: K=%lld not a multiple of 8", (long long)K);
  XK_REQUIRE(group_size > 0 && K % group_size == 0, "int4: group_size=%d does not divide K",
             group_size);
  XK_REQUIRE(E <= 65535 && N < (int64_t(1) << 30) && K < (int64_t(1) << 30), "int4: size limit");
  const int64_t numel = M * top_k;
  XK_REQUIRE(numel < (int64_t(1) << 30), "int4: M*top_k too large");
  if (numel == 0) return XK_OK;
  const Int4Kernel kern = int4_choose(M, top_k, E, N, K, a_dtype, group_size, flags, ep_global);
  // the decode kernel routes for itself when no align outputs are given
  const bool self_route = kern == Int4Kernel::kRs && sorted_ids == nullptr && offsets == nullptr &&
                          int4_rs_self_route_ok(numel);
  if (kern != Int4Kernel::kSimple) {
    XK_REQUIRE(self_route || (sorted_ids && offsets),
               "int4: the MFMA kernels need the align outputs");
    XK_REQUIRE(reinterpret_cast<uintptr_t>(A) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(packed) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(scale) % 16 == 0,
               "int4: A, packed weights and scales must be 16-byte aligned");
  }
  switch (kern) {
    case Int4Kernel::kTile:
      // the tile queue lives in the workspace; without one the tiles are
      // dealt statically
      return launch_int4_prefill(
          A, K, packed, scale, E, N, numel, top_k, group_size, sorted_ids, offsets, slot_out,
          workspace != nullptr && workspace_bytes >= int4_prefill_queue_bytes() &&
                  reinterpret_cast<uintptr_t>(workspace) % 4 == 0
              ? static_cast<int*>(workspace)
              : nullptr,
          stream);
    case Int4Kernel::kRs:
      return launch_int4_rs(A, a_dtype == XK_DT_FP32, M, K, packed, scale, E, N, numel, top_k,
                            group_size, sorted_ids, offsets, topk_ids, emap, num_global, slot_out,
                            stream);
    case Int4Kernel::kSimple:
      break;
  }
  const int64_t total = numel * N;
  const dim3 grid(static_cast<unsigned>(cdiv(total, 256)));
  if (a_dtype == XK_DT_BF16)
    hipLaunchKernelGGL((int4_simple_gemm<uint16_t>), grid, dim3(256), 0, stream,
                       static_cast<const uint16_t*>(A), int(K),
                       reinterpret_cast<const uint32_t*>(packed), scale, int(N), group_size,
                       topk_ids, emap, num_global, int(E), int(numel), int(top_k), slot_out);
  else
    hipLaunchKernelGGL((int4_simple_gemm<float>), grid, dim3(256), 0, stream,
                       static_cast<const float*>(A), int(K),
                       reinterpret_cast<const uint32_t*>(packed), scale, int(N), group_size,
                       topk_ids, emap, num_global, int(E), int(numel), int(top_k), slot_out);
  XK_CHECK_LAUNCH("int4_simple_gemm");
  return XK_OK;
}

}  // namespace xk
