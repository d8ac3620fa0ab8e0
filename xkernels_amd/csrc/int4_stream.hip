// INT4 W4A16 decode-regime grouped GEMM for gfx950 with the reference's
// bf16-rounded weights: the _fused_moe_int4_kernel of
// src/xkernels/ops/moe/triton/moe_int4_kernel.py:78-272, math of the oracle
// reference.py:22-70 with the dequant of w4a16.py:21-50
// (W = bf16((nibble - 8) * scale), then an fp32-accumulated contraction).
//
// Decode experts hold ~11 routed rows, so every packed weight byte feeds one
// 16-row MFMA tile and the kernel is a weight stream (792 MB at the headline
// shape) with ~2.1 VALU instructions of exact dequant per weight. Measured on
// MI355X, that VALU hides only partly under the stream (at the headline shape:
// loads alone 139 us, the whole kernel 164-168 us, a plain read of the same
// bytes ~128 us), so the design removes every other cost from the stream and
// keeps the dequant at its minimum. The same stream serves MXFP4 weights
// (mxfp4_stream_rs below):
//   * work item = (expert, 16-row pass, K slice, 32 output columns). K is cut
//     into S slices only as far as one slice of the pass's activations fits
//     the LDS (S = 2 at K = 7168); every slice writes its own fp32 partial
//     plane (plain stores, summed by the combine in a fixed order), so no
//     workgroup ever switches slices inside a segment;
//   * the items of all experts are split evenly over one 8-wave workgroup per
//     CU (every CU streams the same number of weight bytes); a workgroup's
//     contiguous range holds one or two (expert, pass, slice) segments;
//   * the segment's activations (16 rows x K / S bf16, 112 KiB) are loaded
//     once into LDS by direct-to-LDS loads, already in MFMA operand order (a
//     1 KiB operand is one ds_read_b128 at lane * 16, conflict-free), in
//     natural k order, which is the order dequant_rne_nat emits; rows of pad
//     slots are not read;
//   * each wave streams its column pairs with no barrier: a ring of lines
//     (4 x 16-byte weight loads per 128-byte line of 32 columns) in flight,
//     one line dequantised and contracted per step; the two waves of a SIMD
//     trade issue priority by the steps each has left, so they end together;
//   * group scales come in 8-line blocks: on a block's first line, four loads
//     read 128 contiguous bytes of every column (lane (c, q): lines + q and
//     + q + 4), the wave parks them in a private 4 KiB LDS area and each step
//     reads its own line there. A scale load per line instead (16 columns x
//     16 bytes per instruction, every step) costs ~12 us more at the headline
//     shape: the per-instruction spread over 16 columns, not the bytes, is
//     what counts; 8 rather than 4 lines fetch each 128-byte line of scales
//     once instead of twice (L2 evicts it between the two halves);
//   * lane (c, q) of a load reads bytes 64 h + 16 q of column c's line: the
//     whole quantisation group 4 h + q, one contiguous 64-byte half line per
//     column and instruction. Word j of it feeds MFMA j, so an MFMA contracts
//     four groups (one per lane group) and each lane applies its own group's
//     scale during the dequant;
//   * dequant: dequant_rne_nat (int4_common.h), bit-identical to the reference's
//     bf16((n - 8) * s);
//   * without align outputs (sorted_ids == offsets == null, at most
//     kRsMaxSelf routed slots) every workgroup routes for itself: the mapped
//     expert of every slot goes to LDS with a histogram (LDS atomics), and a
//     segment's 16 rows are found by one wave's ballot scan of that list. The
//     rows of an expert then follow ascending slot order, like the align;
//   * fp32 activations (INT4): staged as bf16 pairs hi + lo through registers,
//     weights split exactly into bf16 hi + lo, three MFMAs per fragment.
#include "int4_common.h"

// cache policy of the partial-row stores: nt (this kernel never re-reads them)
constexpr int kRsStorePolicy = 2;

namespace xk {

int device_cu_count();

namespace {

constexpr int kRsWaves = 8;                 // waves per workgroup (one workgroup per CU)
constexpr int kRsThreads = kRsWaves * 64;
constexpr int kRsMaxCp = 3;                 // column pairs per wave per chunk
constexpr int kRsKeep = 9;                  // finished column pairs a wave holds before writing
constexpr int kRsScLines = 8;               // lines per block of group scales
// Weight formats of the stream: the INT4 W4A16 layout (uint4 nibbles, bf16
// group scales, zero point 8) and MXFP4 (e2m1 nibbles, e8m0 group scales).
// Both pack 32 elements of a group into 16 bytes, low nibble first.
constexpr int kFmtInt4 = 0, kFmtFp4 = 1;
// Cost of entering a segment, in items, for the range split (measured best:
// C2 GEMM 172.9 -> 168.3 us at 6 for INT4; C4 136.3 -> 132.3 us at 4 for MXFP4).
template <int FMT> constexpr int kRsSegGap = FMT == kFmtInt4 ? 6 : 4;
template <int FMT> struct RsFmt {
  static constexpr int kScaleBytes = FMT == kFmtInt4 ? 2 : 1;  // per group
  static constexpr int kLinesPerLoad = 16 / (8 * kScaleBytes);  // lines per 16-byte scale load
  static constexpr int kScLoads = kRsScLines / (4 * kLinesPerLoad);  // per lane and column tile
};
constexpr int kRsRing = 2;                    // ring slots: lines k+1 .. k+R-1 in flight while line k computes
constexpr int kRsLdsA = 112 * 1024;         // bytes of LDS for one activation slice
constexpr int kRsMaxE = 512;
constexpr int kRsMaxSelf = 4096;            // routed slots a workgroup can route for itself

struct RsArgs {
  const uint16_t* A;        // [M, K] bf16
  const uint32_t* packed;   // [E, N, K/8]
  const void* scale;        // [E, N, K/32]: bf16 (INT4) or e8m0 bytes (MXFP4)
  const int32_t* sorted_ids;  // align outputs, or both null: route from topk_ids
  const int32_t* offsets;   // [E+1] padded prefix in slots (multiples of 16)
  const int32_t* topk_ids;  // [numel] (self-routing only)
  const int32_t* emap;      // nullable expert map (self-routing only)
  int num_global;
  float* out;               // [S, numel, N] partial planes
  int K, N, E, numel, top_k;
  int a_row_div;            // A row of slot t: t / a_row_div (top_k: token rows; 1: slot rows)
  int slices;               // S: K slices (16 rows x K / S bf16 fit kRsLdsA)
  uint32_t a_bytes;         // bytes of A (buffer resource range)
  int glog;                 // INT4: log2(group size / 32) (GBIG kernels)
};

// s_waitcnt vmcnt(n) as a real instruction the compiler accounts for (gfx9
// encoding: vmcnt bits 3:0 and 15:14, expcnt and lgkmcnt left at their maxima).
#define XK_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | 0x0F70)

// Workgroup barrier that waits for this wave's LDS operations only; the
// weight loads in flight stay in flight.
__device__ __forceinline__ void lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <typename T> __device__ __forceinline__ T uniform(T x) {
  return __builtin_amdgcn_readfirstlane(x);
}

// Buffer descriptor (gfx9 layout: base, num_records, raw 32-bit access) held
// in SGPRs.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4{static_cast<int32_t>(uniform(static_cast<uint32_t>(a))),
               static_cast<int32_t>(uniform(static_cast<uint32_t>(a >> 32))),
               static_cast<int32_t>(uniform(bytes)), 0x00020000};
}

// Direct-to-LDS 16-byte buffer load: lane i's 16 bytes from voff + soff land
// at lds + 16 i. Issued as inline assembly so that the compiler does not make
// unrelated LDS reads wait for it; the kernel waits for these loads itself
// (XK_WAIT_VMCNT) before it reads the buffer.
__device__ __forceinline__ void dma_16(i32x4 rsrc, const void* lds, int voff, int soff) {
  const uint32_t m0 = uniform(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(rsrc), "s"(uniform(soff))
               : "memory", "m0");
}

// f(integral_constant<int, I>) for I = 0 .. N-1: indices that are constants
// before optimisation, so register arrays indexed by them stay in registers.
template <int N, typename F, int I = 0> __device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, F, I + 1>(static_cast<F&&>(f));
  }
}

// 4 x 4 transpose across the four lanes of a quad (lane bits 0-1 = b):
// afterwards lane b holds element b of every lane of its quad, in lane order.
// Two butterfly stages (partners lane ^ 1, then lane ^ 2), one DPP move per
// element pair; value selects keep the vector in registers.
__device__ __forceinline__ f32x4 quad_transpose(f32x4 e) {
  const int b = threadIdx.x & 3;
  auto stage = [&](auto mc, auto ctrl) __attribute__((always_inline)) {
    constexpr int m = decltype(mc)::value;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i & m) continue;
      const bool hi = (b & m) != 0;
      const float lo_v = e[i], hi_v = e[i + m];
      const float send = hi ? lo_v : hi_v;
      const float recv = __int_as_float(__builtin_amdgcn_update_dpp(
          0, __float_as_int(send), decltype(ctrl)::value, 0xF, 0xF, false));
      e[i] = hi ? recv : lo_v;
      e[i + m] = hi ? hi_v : recv;
    }
  };
  stage(std::integral_constant<int, 1>{}, std::integral_constant<int, 0xB1>{});  // quad_perm 1,0,3,2
  stage(std::integral_constant<int, 2>{}, std::integral_constant<int, 0x4E>{});  // quad_perm 2,3,0,1
  return e;
}

// SLD: bytes per block-start scale load. 16 when K is a multiple of 256 and
// every scale row a 16-byte multiple; else (PADK) 4-byte loads, or 2-byte ones
// for an odd number of scales per row: each lies wholly inside or wholly past
// the buffer (a 16-byte load that straddles the end of the scales comes back
// empty, real bytes included) and needs only 4- (2-) byte aligned rows. K not
// a multiple of 256 zero-pads the last line's activations.
// F32A (INT4 only): fp32 activations, whose reference contraction uses the
// exact products (n - 8) s. The activations are staged as a bf16 pair hi + lo
// (A - hi - lo <= 2^-16 |A|), the weights split exactly (dequant_split_nat),
// and three MFMAs per fragment add hi*hi + hi*lo + lo*hi (lo*lo is below
// 2^-16 of the product): about 2^-15 relative error per term, against the
// spec's fp32 tolerance of 1e-3. The two activation planes halve the K a
// slice holds.
// GBIG (INT4): quantisation groups of 64 or 128 (2^glog 32-k chunks share a
// scale). The block-start scale loads then cover 2^glog lines per 16-byte
// piece, and each lane reads its chunk's scale from the staged block as one
// 16-bit LDS read.
template <int FMT, int SLD, bool F32A = false, bool GBIG = false>
__device__ __forceinline__ void stream_body(const RsArgs& p) {
  constexpr bool PADK = SLD != 16;
  using F = RsFmt<FMT>;
  constexpr int SB = F::kScaleBytes;
  __shared__ __attribute__((aligned(16))) u32x4 a_lds[kRsLdsA / 16];
  __shared__ int pref[kRsMaxE + 1];
  __shared__ int row_slot[16];
  __shared__ int cnt[kRsMaxE];
  __shared__ int16_t slot_expert[kRsMaxSelf];
  __shared__ u32x4 sc_lds[kRsWaves][2][kRsScLines * 16];  // per wave: a block of group scales
  __shared__ int left_lds[kRsWaves];  // INT4: steps each wave has left
  int left = 0;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = uniform(tid >> 6);

  const int c16 = lane & 15, q = lane >> 4;
  const int glog = GBIG ? p.glog : 0;  // log2(group size / 32)
  const int K = p.K, N = p.N, E = p.E, G = K >> (5 + glog), KW = K >> 3;
  // K is cut into 256-k lines, the last one zero-padded when K % 256 != 0
  const int S = p.slices, nl = ((K + 255) >> 8) / S, Ks = nl << 8;
  const bool paired = S > 1 && gridDim.x % (8 * S) == 0;
  const int ncp = (N + 31) >> 5;     // column pairs per expert (N % 32 == 16: the last one half)
  const int nblk = nl * 8;           // 1 KiB operand blocks of one activation slice
  const uint32_t kNibMask = in_vgpr(0x000F000Fu), kNibMaskHi = in_vgpr(0x00F000F0u);

  // Items per expert: 16-row passes x slices x column pairs. Prefix by wave
  // 0 into LDS; the 16-row pass count comes from the align offsets or, when
  // routing here, from an LDS histogram of the mapped experts.
  const bool self_route = p.offsets == nullptr;
  if (self_route) {
    for (int e = tid; e < E; e += kRsThreads) cnt[e] = 0;
    __syncthreads();
    for (int i = tid; i < p.numel; i += kRsThreads) {
      const int e = map_expert(p.topk_ids[i], p.emap, p.num_global, E);
      slot_expert[i] = e;
      if (e >= 0) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
  }
  if (wave == 0) {
    int run = 0;
    for (int base = 0; base < E; base += 64) {
      const int e = base + lane;
      int passes = 0;
      if (e < E) passes = self_route ? (cnt[e] + 15) >> 4 : (p.offsets[e + 1] - p.offsets[e]) >> 4;
      int x = passes * (paired ? 1 : S) * ncp;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
      }
      if (e < E) pref[e + 1] = run + x;
      run += __shfl(x, 63);
    }
    if (lane == 0) pref[0] = 0;
  }
  __syncthreads();
  // Item ranges. Paired (S > 1, grid a multiple of 8 S): the workgroups
  // b, b + 8, ..., b + 8 (S - 1) run on one XCD (workgroups are dealt to the
  // 8 XCDs round-robin) and stream slices 0 .. S-1 of the same range of
  // (expert, pass, column pair) items side by side, so the L2 lines of group
  // scales that straddle a slice boundary (a column's scale row is K / 16
  // bytes, not a multiple of 128) are fetched once for both. Otherwise the
  // items (expert, pass, slice, column pair) are split over the workgroups.
  // Either way a segment (one expert pass and slice) is a run of ncp items,
  // and a range that enters a segment pays its activation load and row scan
  // (about kRsSegGap items' time). The ranges split a cost axis on which
  // every segment is preceded by kRsSegGap virtual items, so a range that
  // crosses into a second segment holds that many fewer real items.
  const int total_items = uniform(pref[E]);
  const int b = blockIdx.x;
  const int gsz = paired ? static_cast<int>(gridDim.x) / S : static_cast<int>(gridDim.x);
  const int grp = paired ? (b / (8 * S)) * 8 + (b & 7) : b;
  const int s_fixed = paired ? (b >> 3) % S : 0;
  const int seg_cost = ncp + kRsSegGap<FMT>;
  const int64_t cost_total = static_cast<int64_t>(total_items / ncp) * seg_cost;
  auto item_at = [&](int64_t v) {  // first real item at or after cost v
    const int64_t sg = v / seg_cost, off = v - sg * seg_cost;
    return static_cast<int>(sg * ncp + (off > kRsSegGap<FMT> ? off - kRsSegGap<FMT> : 0));
  };
  int item_beg, item_end;
  if (cost_total < (int64_t(1) << 30)) {
    // 32-bit divisions (the 64-bit ones cost ~0.5 us at the workgroup's start):
    // with cost_total = cq gsz + cr, cost_total g / gsz = cq g + cr g / gsz
    const int ct = static_cast<int>(cost_total), cq = ct / gsz, cr = ct - cq * gsz;
    auto item_at32 = [&](int v) {
      const int sg = v / seg_cost, off = v - sg * seg_cost;
      return sg * ncp + (off > kRsSegGap<FMT> ? off - kRsSegGap<FMT> : 0);
    };
    item_beg = item_at32(cq * grp + cr * grp / gsz);
    item_end = item_at32(cq * (grp + 1) + cr * (grp + 1) / gsz);
  } else {
    item_beg = item_at(cost_total * grp / gsz);
    item_end = item_at(cost_total * (grp + 1) / gsz);
  }
  // The expert whose items hold position pos: the largest e with pref[e] <= pos
  // (experts without items share their prefix with the next one), counted by
  // one ballot per 64 experts.
  auto expert_of = [&](int pos) __attribute__((always_inline)) {
    int n = 0;
    for (int base = 1; base < E; base += 64) {
      const int e = base + lane;
      n += __popcll(__ballot(e < E && pref[e] <= pos));
    }
    return uniform(n);
  };

  const int w_lane = c16 * KW * 4 + q * 16;  // bytes; + 64 h: group 4 h + q of the line
  const int s_lane = c16 * G * SB;           // bytes: start of column c16's scale row
  // v_perm_b32 selector: bytes 2q, 2q+1 of a scale word pair -> bits 16-31
  const uint32_t s_sel = ((2u * q + 1) << 24) | ((2u * q) << 16) | 0x0C0Cu;
  const i32x4 ra = make_rsrc(p.A, p.a_bytes);
  const int64_t plane = static_cast<int64_t>(p.numel) * N;

  // INT4: the two waves of a SIMD (w and w ^ 4) finish together when the
  // one with more steps left gets the issue priority; without it the older
  // wave wins the arbitration and the younger one runs its last pairs alone
  // (C2 per-wave end times 114 vs 144 us; GEMM 166.5 -> 161.8 us). Each wave
  // first counts the steps of its share (the same walk as the main one, no
  // loads), while the first segment's loads are in flight.
  auto count_steps = [&]() __attribute__((always_inline)) {
  if constexpr (FMT == kFmtInt4) {
    int rot2 = 0, pos2 = item_beg;
    while (pos2 < item_end) {
      const int e = expert_of(pos2);
      const int local = pos2 - pref[e];
      const int cp0 = local % ncp;
      const int cpe = min(ncp, cp0 + (item_end - pos2));
      for (int c0 = cp0; c0 < cpe; c0 += kRsWaves * kRsMaxCp) {
        const int lc = min(kRsWaves * kRsMaxCp, cpe - c0);
        const int base = lc / kRsWaves, rem = lc % kRsWaves;
        const int r = (wave - rot2 + kRsWaves) % kRsWaves;
        const int cnt = base + (r < rem ? 1 : 0);
        if (cnt > 0) left += (cnt * nl + kRsRing - 1) / kRsRing * kRsRing;
        rot2 = (rot2 + rem) % kRsWaves;
      }
      pos2 += cpe - cp0;
    }
    left_lds[wave] = left;  // read after the first segment's barrier
  }
  };

  // Activation slice of a segment -> LDS, in operand order: 1 KiB block
  // blk = (line * 2 + h) * 4 + j holds, at lane qq * 16 + r, the 8 values
  // k = s Ks + line * 256 + (4 h + qq) * 32 + 8 j .. + 7 of row r, in k
  // order. Rows of pad slots read token 0 (never stored).
  // `first`: the workgroup's first segment; each wave counts its steps while
  // the activation loads are in flight. (Pulling the first weight lines of
  // each wave into L2 meanwhile, by direct-to-LDS loads into its scale area,
  // measured slower: the headline GEMM 166 -> 168 / 169 / 170 us at 2 / 3 / 4
  // lines per wave.)
  auto load_segment = [&](int e, int pass, int s, bool first) __attribute__((always_inline)) {
    lds_sync();  // every wave is done with the previous segment
    int sid;
    if (self_route) {
      // rows pass*16 .. +15 of expert e: its slots in ascending order
      if (wave == 0) {
        const int first = pass * 16;
        if (lane < 16) row_slot[lane] = -1;
        int seen = 0;
        for (int i0 = 0; i0 < p.numel && seen < first + 16; i0 += 64) {
          const int i = i0 + lane;
          const bool hit = i < p.numel && slot_expert[i] == e;
          const uint64_t m = __ballot(hit);
          const int rank = seen + __popcll(m & ((uint64_t(1) << lane) - 1));
          if (hit && rank >= first && rank < first + 16) row_slot[rank - first] = i;
          seen += __popcll(m);
        }
      }
      lds_sync();
      sid = row_slot[c16];
    } else {
      const int row0 = uniform(p.offsets[e] + pass * 16);
      if (tid < 16) {
        const int t = p.sorted_ids[row0 + tid];
        row_slot[tid] = t < p.numel ? t : -1;
      }
      const int t = p.sorted_ids[row0 + c16];
      sid = t < p.numel ? t : -1;
    }
    if constexpr (F32A) {
      lds_sync();  // the row table is complete
      const float* A32 = reinterpret_cast<const float*>(p.A);
      // four blocks per thread in flight: their loads issue before any use
      const int total = nblk * 64;
      for (int t0 = tid; t0 < total; t0 += 4 * kRsThreads) {
        f32x4 xs[4][2];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int t = t0 + u * kRsThreads;
          const int blk = t >> 6, ln = t & 63, qq = ln >> 4;
          const int j = blk & 3, h = (blk >> 2) & 1, line = blk >> 3;
          const int k0 = s * Ks + line * 256 + (4 * h + qq) * 32 + 8 * j;
          const int slot = t < total ? row_slot[ln & 15] : -1;
          xs[u][0] = xs[u][1] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (slot >= 0 && k0 < K) {
            const float* a = A32 + static_cast<int64_t>(slot / p.a_row_div) * K + k0;
            xs[u][0] = *reinterpret_cast<const f32x4*>(a);
            xs[u][1] = *reinterpret_cast<const f32x4*>(a + 4);
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int t = t0 + u * kRsThreads;
          if (t >= total) break;
          const float x[8] = {xs[u][0][0], xs[u][0][1], xs[u][0][2], xs[u][0][3],
                              xs[u][1][0], xs[u][1][1], xs[u][1][2], xs[u][1][3]};
          u32x4 vh, vl;
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            typedef float f2 __attribute__((ext_vector_type(2)));
            typedef __bf16 b2 __attribute__((ext_vector_type(2)));
            const uint32_t hh = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{x[2 * e2], x[2 * e2 + 1]}), b2));
            const float r0 = x[2 * e2] - __uint_as_float(hh << 16);
            const float r1 = x[2 * e2 + 1] - __uint_as_float(hh & 0xFFFF0000u);
            vh[e2] = hh;
            vl[e2] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{r0, r1}), b2));
          }
          a_lds[t] = vh;
          a_lds[total + t] = vl;
        }
      }
      if (first) count_steps();
      lds_sync();
      return;
    }
    // rows of pad slots read nothing (an offset past A; their LDS rows only
    // feed output rows that are never stored)
    const int a_voff = sid >= 0 ? (sid / p.a_row_div) * K * 2 + q * 64 : (1 << 30);
    for (int blk = wave; blk < nblk; blk += kRsWaves) {
      const int j = blk & 3, h = (blk >> 2) & 1, line = blk >> 3;
      dma_16(ra, &a_lds[blk * 64], a_voff, (s * Ks + line * 256 + 128 * h + 8 * j) * 2);
    }
    if (first) count_steps();  // while the loads are in flight
    XK_WAIT_VMCNT(0);
    lds_sync();
    if constexpr (PADK) {
      if (s * Ks + Ks > K) {
        // the slice runs past K: its activations there are zero (the weights
        // and scales the stream reads there are finite: other columns' data,
        // or zero past the buffer), after every wave's loads have landed
        for (int t = tid; t < nblk * 64; t += kRsThreads) {
          const int blk = t >> 6, qq = (t & 63) >> 4;
          const int j = blk & 3, h = (blk >> 2) & 1, line = blk >> 3;
          if (s * Ks + line * 256 + (4 * h + qq) * 32 + 8 * j >= K) a_lds[t] = u32x4{0u, 0u, 0u, 0u};
        }
        lds_sync();
      }
    }
  };

  // One chunk: this wave's `cnt` column pairs from `my_lo` of expert e,
  // slice s, each nl lines; results to plane s.
  // Finished column pairs stay in registers (up to kRsKeep per wave) and are
  // written after the wave's stream: writes interleaved with the read stream
  // cost about their own read time again (17.7 MB of partial rows: 17 us at
  // C2), a burst at the end costs their write time. After a quad transpose
  // lane (qa, qb, q) holds row 4 q + qb, columns 4 qa .. 4 qa + 3 of each
  // 16-column tile: two 16-byte stores per kept pair, through a buffer
  // resource (a dropped row's offset lies past the planes).
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      p.out, 0, static_cast<int>(plane * 4 * S), 0x00020000);
  constexpr uint32_t kDrop = 0x80000000u;
  const int qb = lane & 3, qa = (lane >> 2) & 3;  // c16 = 4 qa + qb
  f32x4 keep[kRsKeep][2];
  uint32_t keep_off[kRsKeep];
  // bit i: kept pair i's second 16-column tile lies inside N (N % 32 == 16
  // runs the PADK variants, which keep this mask)
  uint32_t keep_t1 = 0;
  int nkeep = 0;  // wave-uniform
  auto write_kept = [&]() __attribute__((always_inline)) {
    static_for<kRsKeep>([&](auto I) {
      if (decltype(I)::value < nkeep) {
        const f32x4 d0 = quad_transpose(keep[I][0]), d1 = quad_transpose(keep[I][1]);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, d0), ro, keep_off[I], 0,
                                               kRsStorePolicy);
        if (!PADK || ((keep_t1 >> decltype(I)::value) & 1u))
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, d1), ro, keep_off[I] + 64, 0,
                                                 kRsStorePolicy);
      }
    });
    nkeep = 0;
  };

  auto run_chunk = [&](int e, int s, int my_lo, int cnt) __attribute__((always_inline)) {
    if (cnt == 0) return;
    // the chunk's cnt <= kRsMaxCp pairs join the kept ones: room is made
    // before its stream starts, so the step loop below never stores
    if (nkeep + cnt > kRsKeep) write_kept();
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(p.packed + static_cast<int64_t>(e) * N * KW), 0, N * KW * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(static_cast<const uint8_t*>(p.scale) + static_cast<int64_t>(e) * N * G * SB), 0,
        N * G * SB, 0x00020000);
    // Steps (lines) of the chunk, padded to a multiple of kRsRing with dummy
    // steps that re-load the last line and compute nothing, so that the
    // steady-state loop issues every load unconditionally.
    const int steps = cnt * nl;
    const int padded = (steps + kRsRing - 1) / kRsRing * kRsRing;
    int pst = 0, pi = 0, pl = 0;  // prefetch cursor: step, pair, line
    int cst = 0, ci = 0, cl = 0;  // compute cursor

    struct Slot {
      u32x4 w[2][2];  // weights: [column tile][group 4 h + q]
      u32x4 s[2][F::kScLoads];  // block-start steps: scale bytes 16 (q + 4 i) of the block [tile][i]
    };
    Slot rg[kRsRing];
    auto issue = [&](Slot& sl) __attribute__((always_inline)) {
      // Scalar offsets. A load whose scalar offset the compiler cannot prove
      // wave-uniform is wrapped in a loop over lane values: the MXFP4
      // instantiation keeps its cursor in vector registers unless told (INT4
      // keeps it scalar by itself, and there the extra read-first-lane costs
      // vector instructions).
      auto su = [](int x) { return FMT == kFmtInt4 ? x : uniform(x); };
      const int cp = su(my_lo + pi);
      const int wo = su(cp * 32 * KW * 4 + s * (Ks >> 1) + pl * 128);
      const int so = su(cp * 32 * G * SB + ((s * (Ks >> 5) + pl * 8) >> glog) * SB);
      // scales: only on the first line of each block, where lane (c16, q)
      // loads bytes 16 (q + 4 i) .. + 15 of the block's scales (lines pl +
      // (q + 4 i) L .. + L - 1, L = 16-byte loads per line; contiguous bytes
      // per column)
      const bool blk = uniform(((pl & (kRsScLines - 1)) == 0 && pst < steps) ? 1 : 0) != 0;
      const int lines_left = nl - pl;  // scalar: the per-lane test below is one compare
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
          sl.w[c][h] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_lane + 64 * h, wo + c * 16 * KW * 4,
                                                             0);
        if (blk) {  // lanes past the slice's last line read nothing (offset past the buffer)
#pragma unroll
          for (int i = 0; i < F::kScLoads; ++i)
          {
            const int lines = F::kLinesPerLoad << glog;  // lines one 16-byte piece covers
            const bool in = (q + 4 * i) * lines < kRsScLines && (q + 4 * i) * lines < lines_left;
            const int voff = in ? s_lane + 16 * (q + 4 * i) : (1 << 30);
            if constexpr (SLD == 2) {
#pragma unroll
              for (int d = 0; d < 4; ++d) {
                const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(rs, voff + 4 * d, so + c * 16 * G * SB, 0);
                const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(rs, voff + 4 * d + 2, so + c * 16 * G * SB, 0);
                sl.s[c][i][d] = lo | (hi << 16);
              }
            } else if constexpr (SLD == 4) {
#pragma unroll
              for (int d = 0; d < 4; ++d)
                sl.s[c][i][d] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff + 4 * d, so + c * 16 * G * SB,
                                                                     0);
            } else {
              sl.s[c][i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, so + c * 16 * G * SB,
                                                                 0);
            }
          }
        }
      }
      // advance (value selects keep the cursor in scalar registers)
      const int np = pst + 1;
      const int pl1 = pl + (np < steps ? 1 : 0);
      const bool lwrap = pl1 == nl;
      pst = su(np);
      pi = su(pi + (lwrap ? 1 : 0));
      pl = su(lwrap ? 0 : pl1);
    };

    f32x4 acc[2];  // the current column pair's two 16 x 16 tiles
    acc[0] = acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const Slot& sl) __attribute__((always_inline)) {
      const int lbase = cl * (8 * 64) + lane;
      // block start: the loaded scales go to this wave's LDS area (16-byte
      // piece i of the block at 16 i + c16), then every step reads its own
      // line there
      const int lb = cl & (kRsScLines - 1);
      if (lb == 0) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int i = 0; i < F::kScLoads; ++i) sc_lds[wave][c][i * 64 + lane] = sl.s[c][i];
      }
      u32x4 sv[2];     // INT4: the line's 8 bf16 scales
      uint2 sb[2];     // MXFP4: the line's 8 e8m0 bytes
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        if constexpr (FMT == kFmtInt4 && !GBIG)
          sv[c] = sc_lds[wave][c][lb * 16 + c16];
        else
          sb[c] = reinterpret_cast<const uint2*>(&sc_lds[wave][c][0])[((lb >> 1) * 16 + c16) * 2 + (lb & 1)];
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        RneScale ks[2];
        float fs[2];
        bool fnan[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          if constexpr (FMT == kFmtInt4 && GBIG) {  // the bf16 scale of chunk 4 h + q's group
            const int idx = (lb * 8 + 4 * h + q) >> glog;  // scale within the block
            const uint16_t bits =
                reinterpret_cast<const uint16_t*>(&sc_lds[wave][c][0])[((idx >> 3) * 16 + c16) * 8 + (idx & 7)];
            ks[c] = rne_scale(__uint_as_float(uint32_t(bits) << 16));
          } else if constexpr (FMT == kFmtInt4) {  // bf16 scale of group 4 h + q -> fp32 (one v_perm_b32)
            ks[c] = rne_scale(__uint_as_float(__builtin_amdgcn_perm(sv[c][2 * h + 1], sv[c][2 * h], s_sel)));
          } else {  // e8m0 byte of group 4 h + q: byte q of word h
            const uint32_t b = ((h ? sb[c].y : sb[c].x) >> (8 * q)) & 0xFFu;
            fs[c] = e8m0_scale(b);
            fnan[c] = b == 0xFFu;
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bf16x8 bfrag[2];
          [[maybe_unused]] bf16x8 blo[2];
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            if constexpr (F32A)
              dequant_split_nat(sl.w[c][h][j], ks[c], kNibMask, kNibMaskHi, bfrag[c], blo[c]);
            else if constexpr (FMT == kFmtInt4)
              bfrag[c] = dequant_rne_nat(sl.w[c][h][j], ks[c], kNibMask, kNibMaskHi);
            else
              bfrag[c] = fp4x8_to_bf16(fnan[c] ? 0u : sl.w[c][h][j], fs[c]);
          }
          const bf16x8 afrag = __builtin_bit_cast(bf16x8, a_lds[lbase + (h * 4 + j) * 64]);
          if constexpr (F32A) {
            const bf16x8 alo = __builtin_bit_cast(bf16x8, a_lds[nblk * 64 + lbase + (h * 4 + j) * 64]);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, bfrag[c], acc[c], 0, 0, 0);
              acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, blo[c], acc[c], 0, 0, 0);
              acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, bfrag[c], acc[c], 0, 0, 0);
            }
          } else {
#pragma unroll
            for (int c = 0; c < 2; ++c)
              acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, bfrag[c], acc[c], 0, 0, 0);
          }
        }
      }
    };

    // End of a column pair: its partial rows (this slice) join the kept ones.
    auto finish_pair = [&](int i) __attribute__((always_inline)) {
      const int slot = row_slot[4 * q + qb];
      const uint32_t off =
          slot >= 0 ? static_cast<uint32_t>(((s * p.numel + slot) * N + (my_lo + i) * 32 + 4 * qa) * 4)
                    : kDrop;
      // a uniform switch: only the kept slot's registers are written (an
      // unrolled test of every slot compiles to selects over all of them)
      switch (nkeep) {
#define XK_KEEP(I)                                                                              \
  case I:                                                                                       \
    keep[I][0] = acc[0];                                                                        \
    keep[I][1] = acc[1];                                                                        \
    keep_off[I] = off;                                                                          \
    if constexpr (PADK)                                                                         \
      keep_t1 = (keep_t1 & ~(1u << I)) | (((my_lo + i) * 32 + 16 < N ? 1u : 0u) << I);          \
    break;
        XK_KEEP(0) XK_KEEP(1) XK_KEEP(2) XK_KEEP(3) XK_KEEP(4) XK_KEEP(5) XK_KEEP(6) XK_KEEP(7) XK_KEEP(8)
#undef XK_KEEP
        default: break;
      }
      ++nkeep;
      acc[0] = acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // Ring of kRsRing slots: step k issues the loads of step k + kRsRing - 1
    // into the slot freed by step k - 1, then computes step k.
    // (the barriers keep the prologue's slots in issue order: the loop waits
    // for slot 0 first, and a reordered prologue would make it wait for all)
    static_for<kRsRing - 1>([&](auto d) {
      issue(rg[d]);
      __builtin_amdgcn_sched_barrier(0);
    });
    auto step = [&](auto slot) __attribute__((always_inline)) {
      constexpr int nxt = (decltype(slot)::value + kRsRing - 1) % kRsRing;
      issue(rg[nxt]);
      // Dummy steps compute too (after the chunk's last pair, into
      // accumulators that are never kept): every path then consumes the
      // slot's registers, so no temporary aliases a load still in flight and
      // the compiler adds no vmcnt wait that would drain the prefetched lines.
      const bool real = cst < steps;
      compute(rg[slot]);
      const int cl1 = cl + (real ? 1 : 0);
      const bool tend = cl1 == nl;
      if (tend) finish_pair(ci);
      cl = uniform(tend ? 0 : cl1);
      ci = uniform(ci + (tend ? 1 : 0));
      cst = uniform(cst + 1);
      if constexpr (FMT == kFmtInt4) {
        // the wave with more steps left than its SIMD partner issues first
        left_lds[wave] = --left;
        const int other = __builtin_amdgcn_readfirstlane(left_lds[(wave + 4) % kRsWaves]);
        if (other < left)
          __builtin_amdgcn_s_setprio(1);
        else
          __builtin_amdgcn_s_setprio(0);
      }
    };
    for (int st = 0; st < padded; st += kRsRing)
      static_for<kRsRing>([&](auto d) { step(d); });
    // The ring's loads past the last step must land before their registers
    // are reused.
    XK_WAIT_VMCNT(0);
  };

  // Walk this workgroup's item range: segments of one (expert, pass, slice),
  // cut into chunks of at most kRsWaves * kRsMaxCp column pairs.
  int loaded = -1;  // first item of the segment whose activations are in LDS
  int rot = 0;      // first wave to take a remainder pair in the next chunk
  int pos = item_beg;
  while (pos < item_end) {
    const int e = expert_of(pos);
    const int local = pos - pref[e];
    const int seg = local / ncp, cp0 = local - seg * ncp;  // seg = pass (* S + slice)
    const int pass = paired ? seg : seg / S, s = paired ? s_fixed : seg - pass * S;
    const int cpe = min(ncp, cp0 + (item_end - pos));
    const int seg_id = uniform(pos - cp0);
    if (seg_id != loaded) {
      load_segment(e, pass, s, loaded < 0);
      loaded = seg_id;
    }
    for (int c0 = cp0; c0 < cpe; c0 += kRsWaves * kRsMaxCp) {
      const int lc = min(kRsWaves * kRsMaxCp, cpe - c0);
      // lc / 8 pairs each, the remainder to consecutive waves from a rotating
      // start: wave w runs on SIMD w % 4, so the extra pairs spread over the
      // SIMDs and across chunks
      const int base = lc / kRsWaves, rem = lc % kRsWaves;
      const int r = (wave - rot + kRsWaves) % kRsWaves;
      const int my_lo = c0 + r * base + min(r, rem);
      const int cnt = base + (r < rem ? 1 : 0);
      rot = (rot + rem) % kRsWaves;
      run_chunk(e, s, my_lo, cnt);
    }
    pos += cpe - cp0;
  }
  write_kept();
}

__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne(RsArgs p) {
  stream_body<kFmtInt4, 16>(p);
}

// K not a multiple of 256 (a multiple of 64: 4-byte scale rows).
__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_padk(RsArgs p) {
  stream_body<kFmtInt4, 4>(p);
}

// fp32 activations (K a multiple of 256, and the padded variant).
__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_f32(RsArgs p) {
  stream_body<kFmtInt4, 16, true>(p);
}

__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_f32_padk(RsArgs p) {
  stream_body<kFmtInt4, 4, true>(p);
}

// Groups of 64 or 128 (scale rows of 16-byte multiples, K a multiple of 256),
// and the 4-byte-scale-load variants (any even number of scales per row, K a
// multiple of 64).
__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_g(RsArgs p) {
  stream_body<kFmtInt4, 16, false, true>(p);
}

__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_g_padk(RsArgs p) {
  stream_body<kFmtInt4, 4, false, true>(p);
}

__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_g_f32(RsArgs p) {
  stream_body<kFmtInt4, 16, true, true>(p);
}

__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_g_f32_padk(RsArgs p) {
  stream_body<kFmtInt4, 4, true, true>(p);
}

// An odd number of scales per row: 2-byte scale loads (K a multiple of 32).
__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_sld2(RsArgs p) {
  stream_body<kFmtInt4, 2>(p);
}

__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_f32_sld2(RsArgs p) {
  stream_body<kFmtInt4, 2, true>(p);
}

__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_g_sld2(RsArgs p) {
  stream_body<kFmtInt4, 2, false, true>(p);
}

__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
int4_stream_rne_g_f32_sld2(RsArgs p) {
  stream_body<kFmtInt4, 2, true, true>(p);
}

// The same stream over MXFP4 weights (e2m1 nibbles, one e8m0 scale byte per
// 32-element group: 2^(b - 127), byte 0xFF read as 0): each 8-nibble word
// becomes 8 bf16 with four v_cvt_scalef32_pk_bf16_fp4 (exact: an e2m1 value
// times a power of two). Used for both MXFP4 MoE projections, whose fp32
// partial planes are finished by the activation and combine kernels.
__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
mxfp4_stream_rs(RsArgs p) {
  stream_body<kFmtFp4, 16>(p);
}

// K not a multiple of 256 (a multiple of 128: 4-byte scale rows).
__global__ void __launch_bounds__(kRsThreads)
__attribute__((amdgpu_waves_per_eu(kRsWaves / 4, kRsWaves / 4)))
mxfp4_stream_rs_padk(RsArgs p) {
  stream_body<kFmtFp4, 4>(p);
}

}  // namespace

// K slices for one 16-row pass: the fewest (the ceil(K / 256) lines split
// evenly) whose activation block fits the LDS buffer (two bf16 planes for
// fp32 activations). K must be a multiple of the 32-element group.
int rs_slices(int64_t K, bool f32a) {
  if (K % 32 != 0 || K <= 0) return 0;
  const int64_t lines = (K + 255) / 256;  // the last one zero-padded
  const int64_t bytes = f32a ? 4 : 2;
  for (int64_t s = 1; s <= lines; ++s)
    if (lines % s == 0 && 16 * (lines / s) * 256 * bytes <= kRsLdsA) return static_cast<int>(s);
  return 0;
}

// K slices of a stream launch: the fewest the LDS allows. More slices for the
// work balance of small batches measured slower (INT4: the headline shape at
// 4 slices 180 vs 172 us, the N = 7168, K = 2048 down projection at 2 slices
// 93 vs 88 us; MXFP4 at E = 256, hidden 4096, ispp 512, top_k 6 per fused
// call: M = 8 56 -> 76 us, M = 16 76.6 -> 96.9 us with up to 16 slices): a
// slice costs its activation loads and partial plane more than the balance
// gains.
int int4_rs_slices(int64_t K, int64_t N, int64_t numel, int64_t E, bool f32a) {
  (void)N; (void)numel; (void)E;
  return rs_slices(K, f32a);
}

int mxfp4_rs_slices(int64_t K, int64_t N, int64_t numel, int64_t E) {
  (void)N; (void)numel; (void)E;
  return rs_slices(K, false);
}

// Quantisation groups of 32, 64 or 128 (the 16-byte scale loads need 8
// scales per row and K a multiple of 256; else 4-byte loads for an even
// number of scales per row, 2-byte loads for an odd one).
bool int4_rs_group_ok(int64_t K, int group_size) {
  return (group_size == 32 || group_size == 64 || group_size == 128) && K % group_size == 0;
}

bool int4_rs_ok(int64_t M, int64_t top_k, int64_t K, int64_t N, int64_t E, bool f32a,
                int group_size) {
  // the last condition: the fp32 partial planes addressable by one buffer resource
  return K % 32 == 0 && int4_rs_group_ok(K, group_size) && N % 16 == 0 && E <= kRsMaxE &&
         rs_slices(K, f32a) > 0 &&
         N * (K / 8) * 4 < (int64_t(1) << 31) && M * K * 4 < (int64_t(1) << 31) &&
         M * top_k * N * 4 * int4_rs_slices(K, N, M * top_k, E, f32a) < (int64_t(1) << 31);
}

bool int4_rs_self_route_ok(int64_t numel) { return numel <= kRsMaxSelf; }

int launch_int4_rs(const void* A, bool f32a, int64_t M, int64_t K, const int32_t* packed,
                   const uint16_t* scale, int64_t E, int64_t N, int64_t numel, int64_t top_k,
                   int group_size, const int32_t* sorted_ids, const int32_t* offsets,
                   const int32_t* topk_ids, const int32_t* emap, int num_global, float* slot_out,
                   hipStream_t stream) {
  const int glog = group_size == 128 ? 2 : group_size == 64 ? 1 : 0;
  RsArgs a{static_cast<const uint16_t*>(A), reinterpret_cast<const uint32_t*>(packed), scale,
           sorted_ids, offsets, topk_ids, emap, num_global, slot_out, int(K), int(N), int(E),
           int(numel), int(top_k), int(top_k), int4_rs_slices(K, N, numel, E, f32a),
           static_cast<uint32_t>(M * K * (f32a ? 4 : 2)), glog};
  const dim3 grid(static_cast<unsigned>(device_cu_count()));
  // 16-byte scale loads when every scale row is a 16-byte multiple and K a
  // multiple of 256, else 4-byte (even scale count per row) or 2-byte ones
  const int64_t G = K / group_size;
  const int sld = K % 256 == 0 && G % 8 == 0 && N % 32 == 0 ? 16 : G % 2 == 0 ? 4 : 2;
  decltype(&int4_stream_rne) kern;
  if (glog == 0)
    kern = f32a ? (sld == 16 ? int4_stream_rne_f32 : sld == 4 ? int4_stream_rne_f32_padk : int4_stream_rne_f32_sld2)
                : (sld == 16 ? int4_stream_rne : sld == 4 ? int4_stream_rne_padk : int4_stream_rne_sld2);
  else
    kern = f32a ? (sld == 16 ? int4_stream_rne_g_f32 : sld == 4 ? int4_stream_rne_g_f32_padk : int4_stream_rne_g_f32_sld2)
                : (sld == 16 ? int4_stream_rne_g : sld == 4 ? int4_stream_rne_g_padk : int4_stream_rne_g_sld2);
  hipLaunchKernelGGL(kern, grid, dim3(kRsThreads), 0, stream, a);
  XK_CHECK_LAUNCH("int4_stream_rne");
  return XK_OK;
}

bool mxfp4_rs_ok(int64_t a_rows, int64_t K, int64_t N, int64_t E, int64_t numel) {
  const int s = K % 128 == 0 ? mxfp4_rs_slices(K, N, numel, E) : 0;  // 4-byte scale rows
  return s > 0 && N % 32 == 0 && E <= kRsMaxE && N * (K / 2) < (int64_t(1) << 31) &&
         a_rows * K * 2 < (int64_t(1) << 31) && numel * N * 4 * s < (int64_t(1) << 31);
}

int launch_mxfp4_rs(const void* A, int64_t a_rows, int64_t K, const uint8_t* w, const uint8_t* ws,
                    int64_t E, int64_t N, int64_t numel, int64_t a_row_div,
                    const int32_t* sorted_ids, const int32_t* offsets, const int32_t* topk_ids,
                    const int32_t* emap, int num_global, float* planes, hipStream_t stream) {
  RsArgs a{static_cast<const uint16_t*>(A), reinterpret_cast<const uint32_t*>(w), ws, sorted_ids,
           offsets, topk_ids, emap, num_global, planes, int(K), int(N), int(E), int(numel), 1,
           int(a_row_div), mxfp4_rs_slices(K, N, numel, E), static_cast<uint32_t>(a_rows * K * 2), 0};
  if (K % 256 == 0)
    hipLaunchKernelGGL(mxfp4_stream_rs, dim3(static_cast<unsigned>(device_cu_count())),
                       dim3(kRsThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(mxfp4_stream_rs_padk, dim3(static_cast<unsigned>(device_cu_count())),
                       dim3(kRsThreads), 0, stream, a);
  XK_CHECK_LAUNCH("mxfp4_stream_rs");
  return XK_OK;
}

}  // namespace xk

