// Prefill-regime grouped INT4 W4A16 MoE GEMM for gfx950 (the reference's
// _fused_moe_int4_kernel at large M, src/xkernels/ops/moe/triton/moe_int4_kernel.py:78-272;
// math of reference.py:22-70 with the dequant of w4a16.py:21-50).
//
// Same contract as the decode stream kernel: for every routed slot t of local
// expert e it writes the un-weighted fp32 row
//   slot_out[t, n] = sum_k A[t / top_k, k] * bf16((nibble(e, n, k) - 8) * scale[e, n, k / 32])
// and the weighted top-k combine runs afterwards.
//
// With hundreds of routed rows per expert the work is contraction bound, so the
// kernel is an MFMA tile GEMM:
//   * a tile is (expert e, 256 consecutive rows of e's padded slot range, 256
//     output columns); tiles are enumerated on the device from the align
//     offsets, so no host synchronisation is needed;
//   * a persistent grid (one workgroup per CU) walks the tiles. Row blocks are
//     ordered by height class (full blocks and tails above 192 rows, then tails
//     of 129-192, 65-128 and at most 64 rows) and dealt round-robin to the 8
//     XCDs (workgroup b runs on XCD b % 8); a block's column tiles are adjacent
//     in its XCD's sequence, so the workgroups running together on an XCD share
//     the row block's activations in that XCD's L2, and every XCD runs its
//     costliest tiles first and its cheapest last;
//   * 8 waves split the 256 columns; each wave owns all 256 rows x 32 columns
//     (16 x 2 tiles of v_mfma_f32_16x16x32_bf16, 128 accumulator registers), so
//     every weight is dequantised by exactly one wave, once per 256 rows. On
//     gfx950 the dequant's VALU work does not overlap the MFMAs of its SIMD, so
//     the rows a dequantised weight serves set the kernel's speed;
//   * per 128-k step the 256 gathered activation rows are staged in LDS (double
//     buffered, one staging register set loaded a step ahead and written after
//     the step's MFMAs) as they are (the dequant emits natural k order). gfx950 serves a 16-byte LDS read for 32 lanes at a time from 128
//     banks, so the 32 lanes (16 rows x 2 lane groups) of one read must hit 32
//     distinct 16-byte bank groups: rows are 288 bytes apart (18 groups) and the
//     16-byte chunk (lane group q, MFMA j) of a row sits at chunk 4j + q, which
//     makes those 32 groups distinct (measured conflict-free);
//   * lane (c, q) of a wave loads 16 bytes = 32 k of its weight row (quantisation
//     group q of the step) directly into registers, two steps ahead, and
//     dequantises each word with the same fp16-magic / fma_mix / RNE sequence as
//     the decode kernel (dequant_rne_nat: results paired in natural k order),
//     which reproduces the reference's bf16-rounded weights bit for bit.
#include <algorithm>
#include <type_traits>

#include "int4_common.h"

namespace xk {
namespace {

constexpr int kPBM = 256;              // routed rows per tile
constexpr int kPBN = 256;              // output columns per tile
constexpr int kPBK = 128;              // k per pipeline step (4 quantisation groups)
constexpr int kWM = 1;                 // waves along the rows
constexpr int kWN = 8;                 // waves along the columns
constexpr int kPWaves = kWM * kWN;
constexpr int kPThreads = kPWaves * 64;
constexpr int kStRows = kPThreads / 16;    // activation rows staged per pass
constexpr int kRT = kPBM / kWM / 16;   // 16-row MFMA tiles per wave
constexpr int kCT = kPBN / kWN / 16;   // 16-column MFMA tiles per wave
constexpr int kPStride = kPBK + 16;    // bf16 per LDS row (72 dwords)
constexpr int kPMaxExperts = 1024;
constexpr int kXcds = 8;               // MI355X: 8 XCDs, workgroups round-robin over them

struct PrefillArgs {
  const uint16_t* A;       // [M, K] bf16
  const uint32_t* packed;  // [E, N, K/8]
  const uint16_t* scale;   // [E, N, K/g] bf16, g = 32 << glog
  const int32_t* sorted_ids;
  const int32_t* offsets;  // [E+1] padded slot prefix
  float* out;              // [numel, N]
  int K, N, numel, top_k, num_experts;
  int glog;                // log2(group size / 32)
  int* queue;              // [kXcds] tiles taken from each XCD's range (zero at launch), or null
  int a_bytes;             // bytes of A
};

// GBIG: groups of 64 or 128 (chunk 4 s + q's scale is scale[(4 s + q) >> glog]);
// a separate instantiation keeps the 32-wide groups' index math shift-free
// (the shift measured +8 M VALU and +2 % time at C5).
template <bool GBIG>
__device__ __forceinline__ void prefill_body(const PrefillArgs& p) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[2][kPBM * kPStride];
  __shared__ int tok_lds[kPBM];
  __shared__ int slot_lds[kPBM];
  __shared__ int mt_prefix[kPMaxExperts + 1];          // class-0 row blocks per expert (prefix)
  __shared__ uint16_t cl_prefix[3][kPMaxExperts + 1];  // experts with a class-1/2/3 tail (prefix)
  __shared__ int tile_lds;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, q = lane >> 4;
  const int wm = wave % kWM, wn = wave / kWM;
  const int glog = GBIG ? p.glog : 0;
  const int K = p.K, N = p.N, KW = K >> 3, G = K >> (5 + glog);
  const int steps = K / kPBK;
  const int NB = N / kPBN;
  const int E = p.num_experts;
  const uint32_t kNibMask = in_vgpr(0x000F000Fu), kNibMaskHi = in_vgpr(0x00F000F0u);

  // Row blocks in classes by height: 0 = full blocks and tails above 192 rows,
  // 1 = tails of 129-192, 2 = 65-128, 3 = at most 64 rows. Blocks are ordered
  // by class, then expert, and dealt round-robin to the XCDs (block b to XCD
  // b % 8, its column blocks consecutive there), so every XCD's sequence runs
  // from the costliest tiles to the cheapest.
  if (wave == 0) {
    int run[4] = {0, 0, 0, 0};
    for (int base = 0; base < E; base += 64) {
      const int e = base + lane;
      const int rws = e < E ? p.offsets[e + 1] - p.offsets[e] : 0;
      const int full = rws / kPBM, tail = rws - full * kPBM;
      int x[4] = {full + (tail > kPBM * 3 / 4), tail > kPBM / 2 && tail <= kPBM * 3 / 4,
                  tail > kPBM / 4 && tail <= kPBM / 2, tail > 0 && tail <= kPBM / 4};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const int y = __shfl_up(x[c], d);
          if (lane >= d) x[c] += y;
        }
        if (e < E) {
          if (c == 0) mt_prefix[e + 1] = run[0] + x[0];
          else cl_prefix[c - 1][e + 1] = static_cast<uint16_t>(run[c] + x[c]);
        }
        run[c] += __shfl(x[c], 63);
      }
    }
    if (lane == 0) {
      mt_prefix[0] = 0;
      cl_prefix[0][0] = cl_prefix[1][0] = cl_prefix[2][0] = 0;
    }
  }
  __syncthreads();
  const int cb1 = mt_prefix[E], cb2 = cb1 + cl_prefix[0][E], cb3 = cb2 + cl_prefix[1][E];
  const int B = cb3 + cl_prefix[2][E];
  const int xcd = blockIdx.x % kXcds, idx = blockIdx.x / kXcds;
  const int per_xcd = gridDim.x / kXcds;
  // tiles of XCD x: its row blocks x, x + 8, ... times the column blocks
  auto xcd_tiles = [&](int x) { return B > x ? (B - x + kXcds - 1) / kXcds * NB : 0; };
  auto xcd_tile = [&](int x, int n) { return (x + kXcds * (n / NB)) * NB + n % NB; };

  // A staging: thread -> (row st_row + kStRows i, global 16-byte chunk st_kv).
  // Global chunk kv lands at LDS chunk (kv & 3) * 4 + (kv >> 2) (an involution),
  // so lane l of a row loads chunk (l & 3) * 4 + (l >> 2) and the row's 16 lanes
  // write consecutive LDS chunks: the lane-order transpose of the reverse
  // assignment (lane l loads chunk l) cost 62.6 M bank-conflict cycles per C5
  // launch, this one none. The two 16-lane halves of each 32-lane LDS write
  // group take rows 8 apart.
  const int st_kv = ((tid & 3) << 2) | ((tid >> 2) & 3), st_g = tid >> 4;
  const int st_row = (st_g & 1) * 8 + ((st_g >> 1) & 7) + 16 * (st_g >> 4);

  // Tile order. With a queue, each workgroup takes the next tile of its XCD's
  // sequence (an atomic per tile, by one thread) and, when that sequence is
  // exhausted, the next tiles of the other XCDs' sequences: workgroups that
  // finish early take over the rest, and every workgroup exits once all
  // sequences are taken. Without one, workgroup idx of an XCD takes tiles idx,
  // idx + per_xcd, ... of its sequence.
  int n_next = idx;
  for (;;) {
    __syncthreads();  // the previous tile is done with tile_lds, slot_lds and a_lds
    if (tid == 0) {
      int tt = -1;
      if (p.queue == nullptr) {
        tt = n_next < xcd_tiles(xcd) ? xcd_tile(xcd, n_next) : -1;
        n_next += per_xcd;
      } else {
        for (int k = 0; k < kXcds && tt < 0; ++k) {
          const int x = (xcd + k) % kXcds;
          const int nx = xcd_tiles(x);
          if (nx > 0) {
            const int n = atomicAdd(&p.queue[x], 1);
            if (n < nx) tt = xcd_tile(x, n);
          }
        }
      }
      tile_lds = tt;
    }
    __syncthreads();
    const int t = tile_lds;
    if (t < 0) break;
    const int rb = t / NB, nb = t - rb * NB;
    int e, row0;
    if (rb < cb1) {
      int lo = 0, hi = E;  // mt_prefix[lo] <= rb < mt_prefix[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (mt_prefix[mid] <= rb) lo = mid; else hi = mid;
      }
      e = lo;
      row0 = p.offsets[e] + (rb - mt_prefix[e]) * kPBM;
    } else {
      const int c = rb < cb2 ? 0 : rb < cb3 ? 1 : 2;
      const int r = rb - (c == 0 ? cb1 : c == 1 ? cb2 : cb3);
      const uint16_t* pre = cl_prefix[c];
      int lo = 0, hi = E;  // pre[lo] <= r < pre[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pre[mid] <= r) lo = mid; else hi = mid;
      }
      e = lo;
      row0 = p.offsets[e] + (p.offsets[e + 1] - p.offsets[e]) / kPBM * kPBM;
    }
    const int rows = min(kPBM, p.offsets[e + 1] - row0);
    const int n0 = nb * kPBN + wn * (kCT * 16);

    if (tid < kPBM) {
      int slot = -1, tok = -1;
      if (tid < rows) {
        const int s = p.sorted_ids[row0 + tid];
        if (s < p.numel) { slot = s; tok = s / p.top_k; }
      }
      slot_lds[tid] = slot;
      tok_lds[tid] = tok;
    }
    __syncthreads();

    // An expert's last row block of at most 192, 128 or 64 rows runs a
    // shorter tile: fewer MFMAs and staging passes, the same dequant.
    auto run_tile = [&](auto rt_c) __attribute__((always_inline)) {
    constexpr int RT = decltype(rt_c)::value;  // 16-row MFMA tiles
    constexpr int kSP = RT * 16 / kStRows;     // staging passes per step
    // Rows without a token read token 0: MFMA rows are independent and those
    // rows are never stored, so every load stays unconditional.
    // Loads go through buffer resources: a per-lane byte offset fixed for the
    // tile and the step's offset in a scalar register (A below 2^31 bytes and
    // one expert's weights below 2^31 bytes, checked by int4_prefill_ok).
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.A), 0, p.a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(p.packed + static_cast<int64_t>(e) * N * KW), 0, N * KW * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.scale + static_cast<int64_t>(e) * N * G), 0, N * G * 2, 0x00020000);
    uint32_t a_off[kSP];
#pragma unroll
    for (int i = 0; i < kSP; ++i) {
      const int tok = max(tok_lds[st_row + kStRows * i], 0);
      a_off[i] = (static_cast<uint32_t>(tok) * static_cast<uint32_t>(K) + st_kv * 8) * 2;
    }
    uint32_t w_off[kCT], s_off[kCT];
#pragma unroll
    for (int c = 0; c < kCT; ++c) {
      const uint32_t n = n0 + 16 * c + c16;
      w_off[c] = (n * KW + q * 4) * 4;
      s_off[c] = (n * G + (q >> glog)) * 2;
    }

    auto load_a = [&](int s, u32x4 (&ar)[kSP]) {
      s = min(s, steps - 1);
#pragma unroll
      for (int i = 0; i < kSP; ++i)
        ar[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[i], s * (kPBK * 2), 0));
    };
    auto store_a = [&](int buf, const u32x4 (&ar)[kSP]) {
#pragma unroll
      for (int i = 0; i < kSP; ++i) {
        // global chunk st_kv = 4 q + j goes to chunk 4 j + q (natural k order
        // inside the chunk: the dequant emits natural order)
        *reinterpret_cast<u32x4*>(
            &a_lds[buf][(st_row + kStRows * i) * kPStride + ((st_kv & 3) * 4 + (st_kv >> 2)) * 8]) = ar[i];
      }
    };
    auto load_w = [&](int s, u32x4 (&w)[kCT], uint32_t (&sv)[kCT]) {
      s = min(s, steps - 1);
#pragma unroll
      for (int c = 0; c < kCT; ++c) {
        w[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, w_off[c], s * (kPBK / 2), 0));
        // chunk 4 s + q's group: (4 s + q) >> glog = s (4 >> glog) + (q >> glog)
        sv[c] = __builtin_amdgcn_raw_buffer_load_b16(rs, s_off[c], s * ((kPBK / 32) >> glog) * 2, 0);
      }
    };

    f32x4 acc[RT][kCT];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int c = 0; c < kCT; ++c) acc[i][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int buf, const u32x4 (&w)[kCT], const uint32_t (&sv)[kCT]) {
      RneScale ks[kCT];
#pragma unroll
      for (int c = 0; c < kCT; ++c) ks[c] = rne_scale(__uint_as_float(sv[c] << 16));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16x8 b[kCT];
#pragma unroll
        for (int c = 0; c < kCT; ++c) b[c] = dequant_rne_nat(w[c][j], ks[c], kNibMask, kNibMaskHi);
        // row tiles in groups of kAG: the next group's operands are read while
        // the current group's MFMAs run (bounds the registers in flight)
        constexpr int kAG = RT < 2 ? RT : 2;
        auto rd = [&](int i) {
          return *reinterpret_cast<const bf16x8*>(
              &a_lds[buf][(wm * RT * 16 + i * 16 + c16) * kPStride + (j * 4 + q) * 8]);
        };
        bf16x8 af[kAG];
#pragma unroll
        for (int u = 0; u < kAG; ++u) af[u] = rd(u);
#pragma unroll
        for (int g = 0; g < RT / kAG; ++g) {
          bf16x8 an[kAG];
          if (g + 1 < RT / kAG) {
#pragma unroll
            for (int u = 0; u < kAG; ++u) an[u] = rd((g + 1) * kAG + u);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < kAG; ++u)
#pragma unroll
            for (int c = 0; c < kCT; ++c)
              acc[g * kAG + u][c] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[u], b[c], acc[g * kAG + u][c], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
          if (g + 1 < RT / kAG) {
#pragma unroll
            for (int u = 0; u < kAG; ++u) af[u] = an[u];
          }
        }
      }
    };

    u32x4 a0[kSP], w0[kCT], w1[kCT];
    uint32_t s0[kCT], s1[kCT];
    // Prologue: A(0) staged, then W(0) and W(1), the loads the loop expects
    // outstanding at its head.
    load_a(0, a0);
    store_a(0, a0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(0, w0, s0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(1, w1, s1);
    __builtin_amdgcn_sched_barrier(0);
    // step s: A(s+1) -> LDS buffer (s+1)&1 (freed by compute(s-1)) from the
    // register set that then takes A(s+3); contract step s; refill the
    // consumed weight registers with W(s+2). Activation and weight loads are
    // thus two steps old when they are used.
    // (scheduling barriers keep the compiler from sinking the activation loads
    // to their use or hoisting the next store's permutes into compute(), either
    // of which would make a step wait for loads issued in the same step)
    auto step = [&](int s, u32x4 (&w)[kCT], uint32_t (&sv)[kCT]) {
      __syncthreads();
      load_a(s + 1, a0);
      __builtin_amdgcn_sched_barrier(0);
      compute(s & 1, w, sv);
      __builtin_amdgcn_sched_barrier(0);
      load_w(s + 2, w, sv);
      __builtin_amdgcn_sched_barrier(0);
      store_a((s + 1) & 1, a0);
    };
    for (int s = 0; s < steps; s += 2) {
      step(s, w0, s0);
      step(s + 1, w1, s1);
    }

#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int slot = slot_lds[wm * RT * 16 + i * 16 + q * 4 + v];
        if (slot < 0) continue;
        float* orow = p.out + static_cast<int64_t>(slot) * N + n0 + c16;
#pragma unroll
        for (int c = 0; c < kCT; ++c) orow[16 * c] = acc[i][c][v];
      }
    };
    if (rows <= kPBM / 4)
      run_tile(std::integral_constant<int, kRT / 4>{});
    else if (rows <= kPBM / 2)
      run_tile(std::integral_constant<int, kRT / 2>{});
    else if (rows <= kPBM * 3 / 4)
      run_tile(std::integral_constant<int, kRT * 3 / 4>{});
    else
      run_tile(std::integral_constant<int, kRT>{});
  }
}

// Zeroes the tile queue before the tile kernel (a kernel, not a memset, so
// that a captured graph holds no memset node).
__global__ void clear_queue(int* q) {
  if (threadIdx.x < kXcds) q[threadIdx.x] = 0;
}

__global__ void __launch_bounds__(kPThreads)
int4_prefill_gemm(PrefillArgs p) {
  prefill_body<false>(p);
}

__global__ void __launch_bounds__(kPThreads)
int4_prefill_gemm_g(PrefillArgs p) {
  prefill_body<true>(p);
}

}  // namespace

int device_cu_count();

// Bytes of the tile kernel's queue (its workspace).
int64_t int4_prefill_queue_bytes() { return kXcds * sizeof(int); }

// Shapes the tile kernel takes: bf16 activations, groups of 32, 64 or 128, K a
// multiple of two steps, N a multiple of the column tile, at most kPMaxExperts
// local experts, A and one expert's packed weights each below 2^31 bytes (the
// reach of a buffer resource's 32-bit offsets).
bool int4_prefill_ok(int a_dtype, int group_size, int64_t M, int64_t K, int64_t N, int64_t E) {
  return a_dtype == XK_DT_BF16 && (group_size == 32 || group_size == 64 || group_size == 128) &&
         K % (2 * kPBK) == 0 && N % kPBN == 0 && E <= kPMaxExperts &&
         M * K * 2 < (int64_t(1) << 31) && N * K / 2 < (int64_t(1) << 31);
}

int launch_int4_prefill(const void* A, int64_t K, const int32_t* packed, const uint16_t* scale,
                        int64_t E, int64_t N, int64_t numel, int64_t top_k, int group_size,
                        const int32_t* sorted_ids, const int32_t* offsets, float* slot_out,
                        int* queue, hipStream_t stream) {
  XK_REQUIRE(reinterpret_cast<uintptr_t>(A) % 16 == 0 && reinterpret_cast<uintptr_t>(packed) % 16 == 0,
             "int4 prefill: A and packed must be 16-byte aligned");
  const int64_t a_bytes = numel / std::max<int64_t>(top_k, 1) * K * 2;
  XK_REQUIRE(a_bytes < (int64_t(1) << 31) && N * K / 2 < (int64_t(1) << 31),
             "int4 prefill: A and one expert's weights must each be below 2^31 bytes");
  if (queue != nullptr) {
    hipLaunchKernelGGL(clear_queue, dim3(1), dim3(64), 0, stream, queue);
    XK_CHECK_LAUNCH("clear_queue");
  }
  PrefillArgs a{static_cast<const uint16_t*>(A), reinterpret_cast<const uint32_t*>(packed), scale,
                sorted_ids, offsets, slot_out, int(K), int(N), int(numel), int(top_k), int(E),
                group_size == 128 ? 2 : group_size == 64 ? 1 : 0, queue, int(a_bytes)};
  // one workgroup per CU, a multiple of the XCD count
  const int cus = device_cu_count();
  const int grid = std::max(kXcds, cus / kXcds * kXcds);
  hipLaunchKernelGGL(a.glog ? int4_prefill_gemm_g : int4_prefill_gemm, dim3(grid), dim3(kPThreads), 0,
                     stream, a);
  XK_CHECK_LAUNCH("int4_prefill_gemm");
  return XK_OK;
}

}  // namespace xk
