// extern "C" entry points of libxk_moe.so (declared in include/xk_moe.h).
//
// Argument checks happen here, before any launch, so a bad shape is reported as
// XK_ERR_INVALID instead of reaching a kernel. Pipelines carve their scratch
// from the caller's workspace; nothing is allocated here. The one exception to
// "the caller brings the workspace" is xk_moe_int4_w4a16_noalloc, whose scratch
// is a fixed device array of this library (see below).
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>

#include "common.h"
#include "int4_flags.h"

namespace xk {

namespace {
thread_local char g_err[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}
void clear_error() { g_err[0] = '\0'; }

// kernels (align.hip, reduce.hip, int4_gemm.hip, mxfp4_gemm.hip)
int64_t align_workspace_bytes(int64_t numel, int num_experts);
int launch_align(const int32_t* ids, int64_t numel, int num_experts, int block_size,
                 const int32_t* emap, int num_global, int32_t* sorted_ids, int32_t* expert_ids,
                 int32_t* num_post, int32_t* expert_offsets, void* workspace,
                 int64_t workspace_bytes, hipStream_t stream);
int launch_sum_reduce(const void* y, int y_dtype, int64_t M, int64_t top_k, int64_t H,
                      const void* w, int w_dtype, float scale, void* out, hipStream_t stream);
int launch_topk_combine(const float* slot_out, int64_t M, int64_t top_k, int64_t N,
                        const float* topk_w, int mul_routed_weight, const int32_t* topk_ids,
                        int num_local, const int32_t* emap, int num_global, void* out,
                        int out_dtype, int nparts, hipStream_t stream,
                        const uint16_t* post_bias = nullptr, int post_round = 0);
int int4_gemm_parts(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K, int a_dtype,
                    int group_size, int flags, int64_t ep_global = 0);
int int4_block_size();
int int4_kernel_code(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K, int a_dtype,
                     int group_size, int flags, int64_t ep_global);
bool int4_use_stream(int a_dtype, int group_size, int64_t K);
bool int4_gemm_self_routes(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K, int a_dtype,
                           int group_size, int flags, int64_t ep_global = 0);
int64_t int4_gemm_workspace_bytes(int64_t M, int64_t K);
int launch_int4_gemm(const void* A, int a_dtype, int64_t M, int64_t K, const int32_t* packed,
                     const uint16_t* scale, int64_t E, int64_t N, int group_size,
                     const int32_t* topk_ids, int64_t top_k, const int32_t* emap,
                     int num_global, const int32_t* sorted_ids, const int32_t* offsets,
                     float* slot_out, int flags, int64_t ep_global, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream);
int topk_softmax_max_experts();
int launch_topk_softmax(const void* logits, int dtype, int64_t M, int64_t E, int64_t k,
                        int renorm, float* w, int32_t* ids, hipStream_t stream);
int mxfp4_block_size();
int launch_mxfp4_stage(int stage, const void* A, int a_dtype, const uint8_t* w,
                       const uint8_t* ws, const uint16_t* bias, int64_t E, int64_t K,
                       int64_t rows, int64_t ncols, const int32_t* sorted_ids,
                       const int32_t* offsets, int64_t numel, int64_t top_k, float limit,
                       uint16_t* act, float* slot_out, hipStream_t stream);
int mxfp4_rs_slices(int64_t K, int64_t N, int64_t numel, int64_t E);
bool mxfp4_rs_ok(int64_t a_rows, int64_t K, int64_t N, int64_t E, int64_t numel);
int launch_mxfp4_rs(const void* A, int64_t a_rows, int64_t K, const uint8_t* w, const uint8_t* ws,
                    int64_t E, int64_t N, int64_t numel, int64_t a_row_div,
                    const int32_t* sorted_ids, const int32_t* offsets, const int32_t* topk_ids,
                    const int32_t* emap, int num_global, float* planes, hipStream_t stream);
bool int4_rs_self_route_ok(int64_t numel);
int launch_mxfp4_swiglu(const float* planes, int S, int64_t numel, int64_t ispp, const uint16_t* b13,
                        const int32_t* topk_ids, const int32_t* emap, int num_global, int num_local,
                        float limit, uint16_t* act, hipStream_t stream);

namespace {

constexpr int64_t kAlign = 256;
int64_t round_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Scratch of one align call: the outputs the GEMMs consume plus the align's own
// grid scratch.
struct AlignScratch {
  int64_t sorted, expert_ids, num_post, offsets, inner, total;
  AlignScratch(int64_t numel, int num_experts, int block_size) {
    const int64_t max_pad = numel + int64_t(num_experts + 1) * (block_size - 1);
    const int64_t max_blocks = cdiv(max_pad, block_size);
    int64_t o = 0;
    sorted = o; o += round_up(max_pad * 4);
    expert_ids = o; o += round_up(max_blocks * 4);
    num_post = o; o += round_up(4);
    offsets = o; o += round_up(int64_t(num_experts + 1) * 4);
    inner = o; o += round_up(align_workspace_bytes(numel, num_experts));
    total = o;
  }
};

template <typename T> T* at(void* base, int64_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}

int check_dtype(int dt, const char* what) {
  if (dt != XK_DT_BF16 && dt != XK_DT_FP32)
    return set_error(XK_ERR_INVALID, "%s: dtype code %d is neither bf16 nor fp32", what, dt);
  return XK_OK;
}

}  // namespace
}  // namespace xk

using namespace xk;

// ---------------------------------------------------------------------------
// xk_moe_int4_w4a16_noalloc: the fused INT4 call for callers that cannot
// allocate. Its scratch is `scratch`, a device array of kNoAllocScratchBytes
// that every GPU this library runs on holds from module load until the process
// ends. In host code `scratch` names a host-side stand-in, so its device
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and only that address is handed to kernels. Nothing in the fused
// pipeline needs the scratch zeroed (align and the GEMM write every element the
// later kernels read), so no clearing launch is made. Calls that overlap on one
// GPU share the array and race.
namespace xk {
namespace {
constexpr int64_t kNoAllocScratchBytes = int64_t(64) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

int noalloc_scratch(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(XK_ERR_LAUNCH, "int4 noalloc: no current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(XK_ERR_LAUNCH, "int4 noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                       dev, hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *ptr = g_scratch_dev[dev];
  return XK_OK;
}
}  // namespace
}  // namespace xk

extern "C" {

const char* xk_last_error(void) { return g_err; }

int xk_abi_version(void) { return 100; }

int64_t xk_moe_align_workspace_bytes(int64_t numel, int32_t num_experts) {
  return align_workspace_bytes(numel, num_experts);
}

int xk_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int32_t num_experts,
                            int32_t block_size, const int32_t* expert_map,
                            int32_t num_global_experts, int32_t* sorted_token_ids,
                            int32_t* expert_ids, int32_t* num_tokens_post_padded,
                            int32_t* expert_offsets, void* workspace, int64_t workspace_bytes,
                            hipStream_t stream) {
  clear_error();
  return launch_align(topk_ids, numel, num_experts, block_size, expert_map, num_global_experts,
                      sorted_token_ids, expert_ids, num_tokens_post_padded, expert_offsets,
                      workspace, workspace_bytes, stream);
}

int xk_moe_sum_reduce(const void* y, int32_t y_dtype, int64_t M, int64_t top_k, int64_t H,
                      const void* w, int32_t w_dtype, float routed_scaling_factor, void* out,
                      hipStream_t stream) {
  clear_error();
  return launch_sum_reduce(y, y_dtype, M, top_k, H, w, w_dtype, routed_scaling_factor, out,
                           stream);
}

int32_t xk_moe_int4_block_size(int64_t M, int64_t top_k, int64_t E) {
  (void)M; (void)top_k; (void)E;
  return int4_block_size();
}

int32_t xk_moe_int4_kernel(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K,
                           int32_t a_dtype, int32_t group_size, int32_t flags,
                           int32_t num_global_experts) {
  return int4_kernel_code(M, top_k, E, N, K, a_dtype, group_size, flags,
                          num_global_experts > E ? num_global_experts : 0);
}

int32_t xk_moe_int4_gemm_parts(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K,
                               int32_t a_dtype, int32_t group_size, int32_t flags) {
  return int4_gemm_parts(M, top_k, E, N, K, a_dtype, group_size, flags);
}

}  // extern "C"

namespace {
// Fused INT4 scratch: the align outputs, the GEMM's own workspace, then the fp32
// partial planes [parts, numel, N] (the rest of the workspace). The planes are
// sized for the largest count any dtype's default kernel choice writes and,
// under an expert map of ep_global > E experts, the expert-parallel choice's.
int64_t int4_fused_planes(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K,
                          int64_t ep_global) {
  int64_t p = std::max(int4_gemm_parts(M, top_k, E, N, K, XK_DT_BF16, 32, 0),
                       int4_gemm_parts(M, top_k, E, N, K, XK_DT_FP32, 32, 0));
  if (ep_global > E)
    p = std::max<int64_t>(p, std::max(int4_gemm_parts(M, top_k, E, N, K, XK_DT_BF16, 32, 0, ep_global),
                                      int4_gemm_parts(M, top_k, E, N, K, XK_DT_FP32, 32, 0, ep_global)));
  return p;
}
int64_t int4_planes_offset(int64_t M, int64_t top_k, int64_t E, int64_t K) {
  AlignScratch al(M * top_k, int(E), int4_block_size());
  return al.total + round_up(int4_gemm_workspace_bytes(M, K));
}
int64_t int4_fused_bytes(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K,
                         int64_t ep_global) {
  return int4_planes_offset(M, top_k, E, K) +
         round_up(int4_fused_planes(M, top_k, E, N, K, ep_global) * M * top_k * N * 4);
}
}  // namespace

extern "C" {

int64_t xk_moe_int4_w4a16_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t N,
                                          int64_t K) {
  return int4_fused_bytes(M, top_k, E, N, K, 0);
}

int64_t xk_moe_int4_w4a16_ep_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t N,
                                             int64_t K, int32_t num_global_experts) {
  return int4_fused_bytes(M, top_k, E, N, K, num_global_experts);
}

int64_t xk_moe_int4_gemm_workspace_bytes(int64_t M, int64_t K) {
  return int4_gemm_workspace_bytes(M, K);
}

int xk_moe_int4_w4a16_gemm(const void* A, int32_t a_dtype, int64_t M, int64_t K,
                           const int32_t* packed, const uint16_t* scale, int64_t E, int64_t N,
                           int32_t group_size, const int32_t* topk_ids, int64_t top_k,
                           const int32_t* expert_map, int32_t num_global_experts,
                           const int32_t* sorted_token_ids, const int32_t* expert_offsets,
                           float* slot_out, int32_t flags, void* workspace,
                           int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  return launch_int4_gemm(A, a_dtype, M, K, packed, scale, E, N, group_size, topk_ids, top_k,
                          expert_map, num_global_experts, sorted_token_ids, expert_offsets,
                          slot_out, flags, 0, workspace, workspace_bytes, stream);
}

int xk_moe_topk_combine(const float* slot_out, int64_t M, int64_t top_k, int64_t N,
                        const float* topk_w, int32_t mul_routed_weight,
                        const int32_t* topk_ids, int32_t num_local_experts,
                        const int32_t* expert_map, int32_t num_global_experts, void* out,
                        int32_t out_dtype, int32_t nparts, hipStream_t stream) {
  clear_error();
  return launch_topk_combine(slot_out, M, top_k, N, topk_w, mul_routed_weight, topk_ids,
                             num_local_experts, expert_map, num_global_experts, out, out_dtype,
                             nparts, stream);
}

int xk_moe_int4_w4a16(const void* A, int32_t a_dtype, int64_t M, int64_t K,
                      const int32_t* packed, const uint16_t* scale, int64_t E, int64_t N,
                      int32_t group_size, const int32_t* topk_ids, const float* topk_w,
                      int64_t top_k, const int32_t* expert_map, int32_t num_global_experts,
                      int32_t mul_routed_weight, int32_t flags, void* out, void* workspace,
                      int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  if (int rc = check_dtype(a_dtype, "int4 A")) return rc;
  XK_REQUIRE(M >= 0 && top_k >= 1 && E >= 1 && N >= 1, "int4: bad sizes M=%lld top_k=%lld E=%lld N=%lld",
             (long long)M, (long long)top_k, (long long)E, (long long)N);
  XK_REQUIRE(out != nullptr || M == 0, "int4: null out");
  XK_REQUIRE(M == 0 || (A && packed && scale && topk_ids), "int4: null input pointer");
  XK_REQUIRE(!mul_routed_weight || topk_w || M == 0, "int4: null topk_w");
  XK_REQUIRE((flags & ~(XK_INT4_TEST_FORCE_TILE | XK_INT4_TEST_FORCE_STREAM)) == 0,
             "int4: unknown flags 0x%x (pass 0)", flags);
  if (M == 0) return XK_OK;
  const int64_t need = xk_moe_int4_w4a16_workspace_bytes(M, top_k, E, N, K);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(XK_ERR_WORKSPACE, "int4: workspace %lld B < %lld B",
                     (long long)workspace_bytes, (long long)need);
  // A batch whose activations the MFMA kernels cannot address (2^31 bytes
  // through buffer offsets) runs as consecutive token chunks of the largest
  // size they take: a token's output depends only on its own slots (each slot
  // row is a fixed-order K sum, the combine sums a token's slots in slot
  // order), so the chunks write what one call would, bit for bit, with the
  // MFMA kernels instead of the scalar one. Each chunk lays out its smaller
  // workspace at the start of this one; the stream orders them.
  if (flags == 0 && int4_kernel_code(M, top_k, E, N, K, a_dtype, group_size, 0, 0) == 0) {
    const int64_t elem = a_dtype == XK_DT_FP32 ? 4 : 2;
    int64_t mc = ((int64_t(1) << 31) - 1) / (K * elem);
    while (mc > 0 && int4_kernel_code(mc, top_k, E, N, K, a_dtype, group_size, 0, 0) == 0) mc /= 2;
    if (mc > 0 && mc < M) {
      for (int64_t m0 = 0; m0 < M; m0 += mc) {
        const int64_t mm = std::min(mc, M - m0);
        if (int rc = xk_moe_int4_w4a16(static_cast<const char*>(A) + m0 * K * elem, a_dtype, mm, K,
                                       packed, scale, E, N, group_size, topk_ids + m0 * top_k,
                                       topk_w != nullptr ? topk_w + m0 * top_k : nullptr, top_k,
                                       expert_map, num_global_experts, mul_routed_weight, flags,
                                       static_cast<char*>(out) + m0 * N * elem, workspace,
                                       workspace_bytes, stream))
          return rc;
      }
      return XK_OK;
    }
  }
  const int64_t numel = M * top_k;
  AlignScratch al(numel, int(E), int4_block_size());
  const int64_t planes_at = int4_planes_offset(M, top_k, E, K);
  float* slot_out = at<float>(workspace, planes_at);
  const int64_t planes_held = (workspace_bytes - planes_at) / (numel * N * 4);
  // Under an expert map the kernel choice counts the slots expected on the
  // local experts (the dense call's rows per expert) when the workspace holds
  // the partial planes of that choice (xk_moe_int4_w4a16_ep_workspace_bytes
  // sizes for it); else, and with the test bits, every slot counts.
  int64_t ep_global = 0;
  if (flags == 0 && expert_map != nullptr && num_global_experts > E &&
      int4_gemm_parts(M, top_k, E, N, K, a_dtype, group_size, 0, num_global_experts) <= planes_held)
    ep_global = num_global_experts;
  const int64_t parts = int4_gemm_parts(M, top_k, E, N, K, a_dtype, group_size, flags, ep_global);
  // the test bits may force a kernel that writes more partial planes than the
  // default choices the workspace is sized for
  XK_REQUIRE(parts <= planes_held,
             "int4: flags=0x%x need %lld partial planes, more than the workspace holds", flags,
             (long long)parts);
  const int32_t* sorted = nullptr;
  const int32_t* offsets = nullptr;
  // the decode kernel routes for itself; the other MFMA kernels take the align
  if (int4_use_stream(a_dtype, group_size, K) &&
      !int4_gemm_self_routes(M, top_k, E, N, K, a_dtype, group_size, flags, ep_global)) {
    int rc = launch_align(topk_ids, numel, int(E), int4_block_size(), expert_map,
                          num_global_experts, at<int32_t>(workspace, al.sorted),
                          at<int32_t>(workspace, al.expert_ids),
                          at<int32_t>(workspace, al.num_post),
                          at<int32_t>(workspace, al.offsets), at<char>(workspace, al.inner),
                          al.total - al.inner, stream);
    if (rc) return rc;
    sorted = at<int32_t>(workspace, al.sorted);
    offsets = at<int32_t>(workspace, al.offsets);
  }
  if (int rc = launch_int4_gemm(A, a_dtype, M, K, packed, scale, E, N, group_size, topk_ids,
                                top_k, expert_map, num_global_experts, sorted, offsets,
                                slot_out, flags, ep_global, at<char>(workspace, al.total),
                                round_up(int4_gemm_workspace_bytes(M, K)), stream))
    return rc;
  return launch_topk_combine(slot_out, M, top_k, N, topk_w, mul_routed_weight, topk_ids,
                             int(E), expert_map, num_global_experts, out, a_dtype,
                             int(parts), stream);
}

// ---------------------------------------------------------------------------
int64_t xk_moe_int4_w4a16_noalloc_max_bytes() { return xk::kNoAllocScratchBytes; }

int xk_moe_int4_w4a16_noalloc(const void* A, int32_t a_dtype, int64_t M, int64_t K,
                              const int32_t* packed, const uint16_t* scale, int64_t E, int64_t N,
                              int32_t group_size, const int32_t* topk_ids, const float* topk_w,
                              int64_t top_k, const int32_t* expert_map,
                              int32_t num_global_experts, int32_t mul_routed_weight,
                              int32_t flags, void* out, hipStream_t stream) {
  clear_error();
  XK_REQUIRE(M >= 0 && top_k >= 1 && E >= 1 && N >= 1 && K >= 1,
             "int4 noalloc: bad sizes M=%lld top_k=%lld E=%lld N=%lld K=%lld", (long long)M,
             (long long)top_k, (long long)E, (long long)N, (long long)K);
  XK_REQUIRE((flags & ~(XK_INT4_TEST_FORCE_TILE | XK_INT4_TEST_FORCE_STREAM)) == 0,
             "int4 noalloc: unknown flags 0x%x (pass 0)", flags);
  if (M == 0) return XK_OK;
  const int64_t need = xk_moe_int4_w4a16_workspace_bytes(M, top_k, E, N, K);
  XK_REQUIRE(need <= xk::kNoAllocScratchBytes,
             "int4 noalloc: the call needs %lld B of scratch, above the fixed %lld B "
             "(use xk_moe_int4_w4a16 with a workspace)",
             (long long)need, (long long)xk::kNoAllocScratchBytes);
  void* ws = nullptr;
  if (int rc = xk::noalloc_scratch(&ws)) return rc;
  return xk_moe_int4_w4a16(A, a_dtype, M, K, packed, scale, E, N, group_size, topk_ids, topk_w,
                           top_k, expert_map, num_global_experts, mul_routed_weight, flags, out,
                           ws, xk::kNoAllocScratchBytes, stream);
}

int xk_moe_topk_softmax(const void* gating_output, int32_t dtype, int64_t M, int64_t E,
                        int64_t topk, int32_t renormalize, float* topk_weights,
                        int32_t* topk_ids, hipStream_t stream) {
  clear_error();
  XK_REQUIRE(dtype == XK_DT_BF16 || dtype == XK_DT_FP32 || dtype == XK_DT_FP16,
             "topk_softmax: dtype code %d is not bf16, fp32 or fp16", dtype);
  XK_REQUIRE(M >= 0 && E >= 1 && E <= topk_softmax_max_experts(),
             "topk_softmax: bad sizes M=%lld E=%lld (1 <= E <= %d)", (long long)M, (long long)E,
             topk_softmax_max_experts());
  XK_REQUIRE(topk >= 1 && topk <= E, "topk_softmax: topk=%lld outside [1, E=%lld]",
             (long long)topk, (long long)E);
  XK_REQUIRE(M * E < (int64_t(1) << 40), "topk_softmax: M*E too large");
  if (M == 0) return XK_OK;
  XK_REQUIRE(gating_output && topk_weights && topk_ids, "topk_softmax: null pointer");
  return launch_topk_softmax(gating_output, dtype, M, E, topk, renormalize != 0, topk_weights,
                             topk_ids, stream);
}

}  // extern "C"

namespace {

// The MXFP4 pipeline: both projections through the stream kernel (bf16
// activations, shapes within its limits), else the per-stage kernels.
// Workspace after the align scratch: act [numel, ispp] bf16, then the down
// projection's rows [S1, numel, hidden] fp32, then (stream path) the gate/up
// planes [S0, numel, 2 ispp] fp32. The slice counts depend on K only, so the
// workspace bytes never decrease with M and a workspace sized for a batch
// serves every smaller one.
int64_t max_plane_rows(int64_t K, int64_t N, int64_t numel, int64_t E) {
  return mxfp4_rs_slices(K, N, numel, E) * numel;
}

constexpr int64_t kMxStreamRowsPerExpert = 20;

struct Mxfp4Plan {
  bool stream;
  int s0, s1;
  int64_t act, down, gu, total;
  Mxfp4Plan(int64_t M, int64_t top_k, int64_t E, int64_t hidden, int64_t ispp, int a_dtype) {
    const int64_t numel = M * top_k;
    AlignScratch al(numel, int(E), mxfp4_block_size());
    // the stream kernels take each expert's weights once per 16-row pass; from
    // ~20 routed rows per expert on average the per-stage kernels (32 rows a
    // pass) are faster (E = 256, hidden 4096, ispp 512: 280.7 vs 338.2 us at
    // 12 rows per expert, 464.6 vs 445.8 us at 24)
    stream = a_dtype == XK_DT_BF16 && numel > 0 && numel < kMxStreamRowsPerExpert * E &&
             mxfp4_rs_ok(M, hidden, 2 * ispp, E, numel) &&
             mxfp4_rs_ok(numel, ispp, hidden, E, numel);
    s0 = stream ? mxfp4_rs_slices(hidden, 2 * ispp, numel, E) : 0;
    s1 = stream ? mxfp4_rs_slices(ispp, hidden, numel, E) : 1;
    act = al.total;
    down = act + round_up(numel * ispp * 2);
    gu = down + round_up((stream ? max_plane_rows(ispp, hidden, numel, E) : numel) * hidden * 4);
    total = gu + round_up(stream ? max_plane_rows(hidden, 2 * ispp, numel, E) * 2 * ispp * 4 : 0);
  }
};

}  // namespace

extern "C" {

int64_t xk_moe_mxfp4_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t hidden,
                                     int64_t ispp) {
  // the larger of the two plans (the activation dtype is not an argument)
  return std::max(Mxfp4Plan(M, top_k, E, hidden, ispp, XK_DT_BF16).total,
                  Mxfp4Plan(M, top_k, E, hidden, ispp, XK_DT_FP32).total);
}

int xk_moe_mxfp4(const void* A, int32_t a_dtype, int64_t M, int64_t hidden, const uint8_t* w13,
                 const uint8_t* w13_scale, const uint8_t* w2, const uint8_t* w2_scale,
                 int64_t E, int64_t ispp, const uint16_t* b13, const uint16_t* b2,
                 float swiglu_limit, int32_t group_size, const int32_t* topk_ids,
                 const float* topk_w, int64_t top_k, const int32_t* expert_map,
                 int32_t num_global_experts, int32_t mul_routed_weight, void* out,
                 void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  if (int rc = check_dtype(a_dtype, "mxfp4 A")) return rc;
  XK_REQUIRE(group_size == 32, "mxfp4: group_size=%d (only the OCP MX block of 32)", group_size);
  XK_REQUIRE(M >= 0 && top_k >= 1 && E >= 1 && hidden >= 32 && ispp >= 32,
             "mxfp4: bad sizes M=%lld top_k=%lld E=%lld hidden=%lld ispp=%lld", (long long)M,
             (long long)top_k, (long long)E, (long long)hidden, (long long)ispp);
  XK_REQUIRE(hidden % 32 == 0 && ispp % 32 == 0, "mxfp4: hidden and ispp must be multiples of 32");
  XK_REQUIRE(M == 0 || (A && w13 && w13_scale && w2 && w2_scale && topk_ids && out),
             "mxfp4: null pointer");
  XK_REQUIRE(!mul_routed_weight || topk_w || M == 0, "mxfp4: null topk_w");
  if (M == 0) return XK_OK;
  const int64_t need = xk_moe_mxfp4_workspace_bytes(M, top_k, E, hidden, ispp);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(XK_ERR_WORKSPACE, "mxfp4: workspace %lld B < %lld B",
                     (long long)workspace_bytes, (long long)need);
  const int64_t numel = M * top_k;
  AlignScratch al(numel, int(E), mxfp4_block_size());
  const Mxfp4Plan plan(M, top_k, E, hidden, ispp, a_dtype);
  uint16_t* act = at<uint16_t>(workspace, plan.act);
  float* slot_out = at<float>(workspace, plan.down);
  int32_t* sorted = at<int32_t>(workspace, al.sorted);
  int32_t* offsets = at<int32_t>(workspace, al.offsets);
  // the stream kernels route small batches themselves (no align kernel)
  const bool self_route = plan.stream && int4_rs_self_route_ok(numel);
  int rc = XK_OK;
  if (!self_route) {
    rc = launch_align(topk_ids, numel, int(E), mxfp4_block_size(), expert_map, num_global_experts,
                      sorted, at<int32_t>(workspace, al.expert_ids),
                      at<int32_t>(workspace, al.num_post), offsets, at<char>(workspace, al.inner),
                      al.total - al.inner, stream);
    if (rc) return rc;
  }
  if (plan.stream) {
    const int32_t* rs_sorted = self_route ? nullptr : sorted;
    const int32_t* rs_offsets = self_route ? nullptr : offsets;
    float* gu = at<float>(workspace, plan.gu);
    rc = launch_mxfp4_rs(A, M, hidden, w13, w13_scale, E, 2 * ispp, numel, top_k, rs_sorted,
                         rs_offsets, topk_ids, expert_map, num_global_experts, gu, stream);
    if (rc) return rc;
    rc = launch_mxfp4_swiglu(gu, plan.s0, numel, ispp, b13, topk_ids, expert_map,
                             num_global_experts, int(E), swiglu_limit, act, stream);
    if (rc) return rc;
    rc = launch_mxfp4_rs(act, numel, ispp, w2, w2_scale, E, hidden, numel, 1, rs_sorted, rs_offsets,
                         topk_ids, expert_map, num_global_experts, slot_out, stream);
    if (rc) return rc;
    return launch_topk_combine(slot_out, M, top_k, hidden, topk_w, mul_routed_weight, topk_ids,
                               int(E), expert_map, num_global_experts, out, a_dtype, plan.s1, stream,
                               b2, 1);
  }
  rc = launch_mxfp4_stage(0, A, a_dtype, w13, w13_scale, b13, E, hidden, 2 * ispp, ispp, sorted,
                          offsets, numel, top_k, swiglu_limit, act, nullptr, stream);
  if (rc) return rc;
  rc = launch_mxfp4_stage(1, act, XK_DT_BF16, w2, w2_scale, b2, E, ispp, hidden, hidden, sorted,
                          offsets, numel, top_k, 0.f, nullptr, slot_out, stream);
  if (rc) return rc;
  return launch_topk_combine(slot_out, M, top_k, hidden, topk_w, mul_routed_weight, topk_ids,
                             int(E), expert_map, num_global_experts, out, a_dtype, 1, stream);
}

}  // extern "C"
