// Grouped INT4 W4A16 MoE GEMM for gfx950 (the reference's _fused_moe_int4_kernel,
// src/xkernels/ops/moe/triton/moe_int4_kernel.py:78-272; math of the oracle
// reference.py:22-70 with the dequant of w4a16.py:21-50).
//
// For every routed slot t (token m = t / top_k, local expert e) this writes the
// un-weighted fp32 row   slot_out[t, n] = sum_k A[m, k] * W[e, n, k]
// with W[e, n, k] = (nibble(e, n, k) - 8) * scale[e, n, k / 32]. The weighted
// top-k combine runs afterwards (reduce.hip).
//
// Two stream kernels (bf16 A, group 32). int4_stream_gemm_rne (default) rounds
// every dequantised weight to bf16 like the reference; int4_stream_gemm
// (XK_INT4_FAST_DEQUANT) is described next.
// Fast stream kernel — the decode regime is weight-streaming
// bound, so every packed weight byte is read from HBM exactly once:
//   * one workgroup owns (expert e, 128 output columns) and ALL of e's slots,
//     taking them 32 at a time, so an expert's weights are streamed once per
//     32 routed slots (decode experts hold ~11);
//   * wave w owns 32 columns = two 16x16 MFMA column tiles; lane (c, q) reads
//     word q of every 32-k group of its column with a 4-byte load, so one
//     v_mfma_f32_16x16x32_bf16 contracts exactly one quantisation group;
//   * nibbles become bf16 (128 + n) with one v_and_or_b32 per two values (the
//     exponent of 128 places the nibble in the mantissa); the MFMA then gives
//     D = sum a*(128+n) and the group result is s * (D - 136 * sum(a)), where
//     sum(a) over the 32 activations of the group is computed once per
//     workgroup while staging A into LDS. The dequantised weight (n-8)*s is
//     exact in fp32 this way; the reference rounds it to bf16 first, a
//     difference far inside the op's 2e-2 tolerance;
//   * A (the expert's activation rows, 32 x 256 k per chunk) is staged in LDS
//     with the same k-permutation the nibble unpack produces, and the next
//     chunk's weights, scales and activations are prefetched into registers
//     while the current chunk is contracted.
// Simple kernel: any dtype / group size, one thread per (slot, column), exact
// dequant rounded to A's dtype like the reference. Correctness fallback for the
// fp32 sweep points and unusual group sizes.
#include <algorithm>
#include <type_traits>

#include "int4_common.h"

#ifndef XK_INT4_STREAM_OCC
#define XK_INT4_STREAM_OCC 2
#endif
#ifndef XK_INT4_STREAM_WAVES
#define XK_INT4_STREAM_WAVES 4
#endif

namespace xk {
namespace {

constexpr int kWaves = 4;
constexpr int kColsPerWave = 32;
constexpr int kColsPerWG = kWaves * kColsPerWave;  // 128
constexpr int kChunkGroups = 8;                    // 8 x 32 k = 256 k per chunk
constexpr int kChunkK = kChunkGroups * 32;
constexpr int kRowsPerPass = 32;                   // two 16-row MFMA tiles
constexpr int kALdsStride = kChunkK + 8;           // bf16 elements, +16 B pad

struct StreamArgs {
  const uint16_t* A;       // [M, K] bf16
  const uint32_t* packed;  // [E, N, K/8]
  const uint16_t* scale;   // [E, N, K/32] bf16
  const int32_t* sorted_ids;
  const int32_t* offsets;  // [E+1] padded prefix (slots), multiples of 16
  float* out;              // [numel, N]
  int K, N, numel, top_k;
  int scale_vec;           // scale rows are 16-byte aligned (K/32 % 8 == 0)
};

__device__ __forceinline__ uint32_t nib_pair(uint32_t w, int shift) {
  // bf16 pair (128 + nibble[d], 128 + nibble[d+4]) for d = shift / 4
  return ((w >> shift) & 0x000F000Fu) | 0x43004300u;
}


__global__ void __launch_bounds__(256)
int4_stream_gemm(StreamArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[kRowsPerPass * kALdsStride];
  __shared__ __attribute__((aligned(16))) float r_lds[kChunkGroups * kRowsPerPass];
  __shared__ int slot_lds[kRowsPerPass];
  __shared__ int tok_lds[kRowsPerPass];

  const int e = blockIdx.y;
  const int beg = p.offsets[e], end = p.offsets[e + 1];
  if (beg >= end) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, q = lane >> 4;
  const int K = p.K, N = p.N, G = K >> 5, KW = K >> 3;
  const int n_base = blockIdx.x * kColsPerWG + wave * kColsPerWave;

  const uint32_t* wrow[2];
  const uint16_t* srow[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int n = min(n_base + 16 * c + c16, N - 1);
    wrow[c] = p.packed + (static_cast<int64_t>(e) * N + n) * KW + q;
    srow[c] = p.scale + (static_cast<int64_t>(e) * N + n) * G;
  }
  // Staging role: thread -> (row r, group gg) of the 32 x 8 activation chunk.
  const int st_r = tid >> 3, st_g = tid & 7;

  for (int pass = beg; pass < end; pass += kRowsPerPass) {
    const int ntiles = min(2, (end - pass) >> 4);
    __syncthreads();  // previous pass finished with slot_lds / tok_lds
    if (tid < kRowsPerPass) {
      int slot = -1, tok = -1;
      if (tid < ntiles * 16) {
        const int s = p.sorted_ids[pass + tid];
        if (s < p.numel) { slot = s; tok = s / p.top_k; }
      }
      slot_lds[tid] = slot;
      tok_lds[tid] = tok;
    }
    __syncthreads();
    const int my_tok = tok_lds[st_r];

    auto load_a = [&](int g0, uint32_t* areg) {
      const int g = g0 + st_g;
      if (my_tok >= 0 && g < G) {
        const u32x4* src = reinterpret_cast<const u32x4*>(
            p.A + static_cast<int64_t>(my_tok) * K + g * 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x4 v = src[j];
#pragma unroll
          for (int i = 0; i < 4; ++i) areg[4 * j + i] = v[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) areg[i] = 0u;
      }
    };
    auto load_w = [&](int g0, uint32_t (*wreg)[kChunkGroups], uint32_t (*sreg)[4]) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int g = 0; g < kChunkGroups; ++g)
          wreg[c][g] = (g0 + g < G) ? wrow[c][(g0 + g) * 4] : 0u;
        if (p.scale_vec) {
          const u32x4 s4 = *reinterpret_cast<const u32x4*>(srow[c] + g0);
#pragma unroll
          for (int i = 0; i < 4; ++i) sreg[c][i] = s4[i];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (g0 + 2 * i < G) ? srow[c][g0 + 2 * i] : 0u;
            const uint32_t hi = (g0 + 2 * i + 1 < G) ? srow[c][g0 + 2 * i + 1] : 0u;
            sreg[c][i] = lo | (hi << 16);
          }
        }
      }
    };

    f32x4 acc[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint32_t areg[16];
    uint32_t wcur[2][kChunkGroups], wnext[2][kChunkGroups];
    uint32_t scur[2][4], snext[2][4];
    load_a(0, areg);
    load_w(0, wcur, scur);

    for (int g0 = 0; g0 < G; g0 += kChunkGroups) {
      __syncthreads();  // all waves done reading the previous chunk
      {
        // write staged activations (k-permuted) and their group sums
        float rs = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i)
          rs += __uint_as_float(areg[i] << 16) + __uint_as_float(areg[i] & 0xFFFF0000u);
        uint32_t o[16];
#pragma unroll
        for (int s = 0; s < 4; ++s) perm8(areg + 4 * s, o + 4 * s);
        u32x4* dst = reinterpret_cast<u32x4*>(a_lds + st_r * kALdsStride + st_g * 32);
#pragma unroll
        for (int s = 0; s < 4; ++s) dst[s] = u32x4{o[4 * s], o[4 * s + 1], o[4 * s + 2], o[4 * s + 3]};
        r_lds[st_g * kRowsPerPass + st_r] = rs;
      }
      __syncthreads();
      const int gn = g0 + kChunkGroups;
      if (gn < G) {
        load_a(gn, areg);
        load_w(gn, wnext, snext);
      }
#pragma unroll
      for (int g = 0; g < kChunkGroups; ++g) {
        if (g0 + g >= G) break;
        bf16x8 bfrag[2];
        float sc[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const uint32_t w = wcur[c][g];
          const u32x4 b = u32x4{nib_pair(w, 0), nib_pair(w, 4), nib_pair(w, 8), nib_pair(w, 12)};
          bfrag[c] = __builtin_bit_cast(bf16x8, b);
          const uint32_t sw = scur[c][g >> 1];
          sc[c] = __uint_as_float((g & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (t >= ntiles) break;
          const bf16x8 afrag = *reinterpret_cast<const bf16x8*>(
              a_lds + (t * 16 + c16) * kALdsStride + g * 32 + q * 8);
          const f32x4 r4 = *reinterpret_cast<const f32x4*>(r_lds + g * kRowsPerPass + t * 16 + q * 4);
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                afrag, bfrag[c], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[t][c][i] = fmaf(sc[c], fmaf(-136.0f, r4[i], d[i]), acc[t][c][i]);
          }
        }
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int g = 0; g < kChunkGroups; ++g) wcur[c][g] = wnext[c][g];
#pragma unroll
        for (int i = 0; i < 4; ++i) scur[c][i] = snext[c][i];
      }
    }

    // epilogue: D row (4q + i) of tile t, column c16 of column tile c
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t >= ntiles) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int slot = slot_lds[t * 16 + q * 4 + i];
        if (slot < 0) continue;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int n = n_base + 16 * c + c16;
          if (n < N) p.out[static_cast<int64_t>(slot) * N + n] = acc[t][c][i];
        }
      }
    }
  }
}

// Reference-faithful stream kernel: each weight is dequantised as
// bf16_rne((n - 8) * s) (v_cvt_f32_ubyte + v_fma_f32 + v_cvt_pk_bf16_f32, the
// reference's w4a16.py:42-50 rounding) before the MFMA, so the contraction sees
// the same bf16 weights the reference multiplies. With the scale applied before
// the MFMA the k order inside an MFMA is free: lane (c, q) loads 16 bytes = one
// whole 32-k group (group g0 + q of the step) and feeds four MFMAs from it.
__global__ void __launch_bounds__(256)
int4_stream_gemm_rne(StreamArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[kRowsPerPass * kALdsStride];
  __shared__ int slot_lds[kRowsPerPass];
  __shared__ int tok_lds[kRowsPerPass];

  const int e = blockIdx.y;
  const int beg = p.offsets[e], end = p.offsets[e + 1];
  if (beg >= end) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, q = lane >> 4;
  const int K = p.K, N = p.N, G = K >> 5, KW = K >> 3;
  const int n_base = blockIdx.x * kColsPerWG + wave * kColsPerWave;

  const uint32_t* wrow[2];
  const uint16_t* srow[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int n = min(n_base + 16 * c + c16, N - 1);
    wrow[c] = p.packed + (static_cast<int64_t>(e) * N + n) * KW;
    srow[c] = p.scale + (static_cast<int64_t>(e) * N + n) * G;
  }
  const int st_r = tid >> 3, st_g = tid & 7;

  for (int pass = beg; pass < end; pass += kRowsPerPass) {
    const int ntiles = min(2, (end - pass) >> 4);
    __syncthreads();
    if (tid < kRowsPerPass) {
      int slot = -1, tok = -1;
      if (tid < ntiles * 16) {
        const int s = p.sorted_ids[pass + tid];
        if (s < p.numel) { slot = s; tok = s / p.top_k; }
      }
      slot_lds[tid] = slot;
      tok_lds[tid] = tok;
    }
    __syncthreads();
    const int my_tok = tok_lds[st_r];

    auto load_a = [&](int g0, uint32_t* areg) {
      const int g = g0 + st_g;
      if (my_tok >= 0 && g < G) {
        const u32x4* src = reinterpret_cast<const u32x4*>(
            p.A + static_cast<int64_t>(my_tok) * K + g * 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x4 v = src[j];
#pragma unroll
          for (int i = 0; i < 4; ++i) areg[4 * j + i] = v[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) areg[i] = 0u;
      }
    };
    // weights of groups g0 + 4h + q (h = 0, 1) for both column tiles
    auto load_w = [&](int g0, u32x4 (*wr)[2], float (*sr)[2]) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int g = g0 + 4 * h + q;
          if (g < G) {
            wr[c][h] = *reinterpret_cast<const u32x4*>(wrow[c] + g * 4);
            sr[c][h] = bf16_to_f32(srow[c][g]);
          } else {
            wr[c][h] = u32x4{0u, 0u, 0u, 0u};
            sr[c][h] = 0.f;
          }
        }
    };

    f32x4 acc[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint32_t areg[16];
    u32x4 wcur[2][2], wnext[2][2];
    float scur[2][2], snext[2][2];
    load_a(0, areg);
    load_w(0, wcur, scur);

    for (int g0 = 0; g0 < G; g0 += kChunkGroups) {
      __syncthreads();
      {
        u32x4* dst = reinterpret_cast<u32x4*>(a_lds + st_r * kALdsStride + st_g * 32);
#pragma unroll
        for (int s = 0; s < 4; ++s)
          dst[s] = u32x4{areg[4 * s], areg[4 * s + 1], areg[4 * s + 2], areg[4 * s + 3]};
      }
      __syncthreads();
      const int gn = g0 + kChunkGroups;
      if (gn < G) {
        load_a(gn, areg);
        load_w(gn, wnext, snext);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (g0 + 4 * h >= G) break;
        // dequantise the four words of both column tiles
        bf16x8 bfrag[2][4];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const float s = scur[c][h], ms = -8.0f * s;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            uint32_t t = wcur[c][h][j] & 0x0F0F0F0Fu;
            uint32_t u = (wcur[c][h][j] >> 4) & 0x0F0F0F0Fu;
            // keep the byte-lane form so each nibble converts with v_cvt_f32_ubyteN
            asm("" : "+v"(t));
            asm("" : "+v"(u));
            u32x4 b;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float lo = fmaf(static_cast<float>((t >> (8 * i)) & 0xFFu), s, ms);
              const float hi = fmaf(static_cast<float>((u >> (8 * i)) & 0xFFu), s, ms);
              b[i] = static_cast<uint32_t>(f32_to_bf16(lo)) |
                     (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
            }
            bfrag[c][j] = __builtin_bit_cast(bf16x8, b);
          }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (t >= ntiles) break;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bf16x8 afrag = *reinterpret_cast<const bf16x8*>(
                a_lds + (t * 16 + c16) * kALdsStride + (4 * h + q) * 32 + 8 * j);
#pragma unroll
            for (int c = 0; c < 2; ++c)
              acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, bfrag[c][j], acc[t][c], 0, 0, 0);
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
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int n = n_base + 16 * c + c16;
          if (n < N) p.out[static_cast<int64_t>(slot) * N + n] = acc[t][c][i];
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------
// Persistent stream kernel (K % 256 == 0), the production decode path. Same
// math as the two kernels above, restructured for bytes in flight:
//   * work items are (active expert, 128-column block); the grid is sized to
//     the machine (2 workgroups per CU) and each workgroup walks items
//     blockIdx.x, blockIdx.x + gridDim.x, ...; the active-expert list is
//     rebuilt per item from the padded offsets with one ballot per 64 experts
//     (no host sync);
//   * every lane loads 16 bytes (one whole 32-k group) per column tile and
//     chunk half, from a 4-deep register ring (weights requested 3 chunks
//     ahead); activations go through two LDS buffers (one barrier per chunk);
//     every global load is unconditional (clamped indices) so the compiler can
//     count outstanding loads instead of draining them;
//   * every load a step consumes (weights of chunk c, activations of chunk
//     c+1, the scale piece of chunk c+8) was issued three steps earlier and in
//     the same step: loads return in issue order, so a wait for a load issued
//     later than the weights it follows would drain the weight ring;
//   * group scales: each wave keeps its 32 rows' scales for 16 chunks in an
//     LDS ring (16 bytes per row and chunk), refilled 8 bytes per lane per
//     step, 8 chunks ahead of use;
//   * activations are staged with the k-permutation the nibble unpack
//     produces and a 544-byte row pitch, so the MFMA operand reads are
//     bank-conflict free;
//   * RNE mode dequantises every weight to bf16_rne((n-8)*s) before the MFMA
//     (reference rounding). FAST mode contracts in fp16 against activations
//     prepared by int4_prep_a (fp16, exact per-row power-of-two scale, the
//     unpack's k order, 1/16 at the 16n positions): it transposes the four
//     words of a group across the four lane groups with v_permlane32_swap /
//     v_permlane16_swap so one MFMA contracts one group, unpacks nibbles to
//     fp16 1024+n / 1024+16n with one v_and_or_b32 per pair, removes the
//     offsets with a second MFMA against a constant operand (shared by both
//     column tiles) and applies the group scale to the MFMA result. The
//     weights are then exact (n-8)*s rather than bf16-rounded.
enum class Int4Mode { kRne, kFast };

constexpr int kV2Rows = 32;  // two 16-row MFMA tiles per pass
constexpr int kV2Stride = kChunkK + 16;  // bf16 per LDS row: 544 B, bank-staggered rows

struct V2Args {
  StreamArgs s;
  int num_experts;
  const int32_t* a_exp;  // FAST: per-token power-of-two exponent of the prepared A
};

template <Int4Mode MODE, int WAVES, int MAXNT>
__global__ void __launch_bounds__(WAVES * 64)
__attribute__((amdgpu_waves_per_eu(XK_INT4_STREAM_OCC, XK_INT4_STREAM_OCC)))
int4_stream_v2(V2Args args) {
  constexpr bool kFast = MODE == Int4Mode::kFast;
  constexpr int kThreads = WAVES * 64;
  constexpr int kCols = WAVES * kColsPerWave;  // output columns per work item
  constexpr int kRing = 4;         // register ring depth (loads issued 3 steps ahead)
  constexpr int kSSlots = 16;      // scale LDS ring: chunks held per row
  constexpr int kSStride = kSSlots * 8 + 8;      // bf16 per scale row in LDS (16 B pad)
  constexpr int kRowsPass = 16 * MAXNT;          // routed rows per pass
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[2][kRowsPass * kV2Stride];
  __shared__ __attribute__((aligned(16))) uint16_t s_lds[WAVES][32 * kSStride];
  __shared__ int slot_lds[kRowsPass];
  __shared__ int tok_lds[kRowsPass];
  __shared__ int exp_lds[kRowsPass];
  const StreamArgs& p = args.s;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, q = lane >> 4;
  const int K = p.K, N = p.N, G = K >> 5, KW = K >> 3;
  const int nb = (N + kCols - 1) / kCols;
  const int nchunks = G / kChunkGroups;
  const int items = count_active_experts(p.offsets, args.num_experts) * nb;
  const uint32_t kNibMask = in_vgpr(0x000F000Fu), kNibMaskHi = in_vgpr(0x00F000F0u);
  typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
  // -1032 at the 1024 + n positions, -1152 (= 16 * 72) at the 1024 + 16n ones
  const f16x8 negc = __builtin_bit_cast(f16x8, u32x4{0xE408E408u, 0xE480E480u, 0xE408E408u, 0xE480E480u});

  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int e = find_active_expert(p.offsets, args.num_experts, item / nb);
    const int n_base = (item % nb) * kCols + wave * kColsPerWave;
    const int beg = p.offsets[e], end = p.offsets[e + 1];
    const uint32_t* wrow[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int n = min(n_base + 16 * c + c16, N - 1);
      wrow[c] = p.packed + (static_cast<int64_t>(e) * N + n) * KW + q * 4;
    }
    // scale pieces: lane -> (row lane/2 of the wave's 32 rows, 8-byte half lane&1)
    const int sp_row = lane >> 1, sp_half = lane & 1;
    const uint16_t* sp_src =
        p.scale + (static_cast<int64_t>(e) * N + min(n_base + sp_row, N - 1)) * G + sp_half * 4;

    for (int pass = beg; pass < end; pass += kRowsPass) {
      const int ntiles = min(MAXNT, (end - pass) >> 4);
      __syncthreads();  // previous pass / item done with LDS
      if (tid < kRowsPass) {
        int slot = -1, tok = -1;
        if (tid < ntiles * 16) {
          const int sidx = p.sorted_ids[pass + tid];
          if (sidx < p.numel) { slot = sidx; tok = sidx / p.top_k; }
        }
        slot_lds[tid] = slot;
        tok_lds[tid] = tok;
        if constexpr (kFast) exp_lds[tid] = tok >= 0 ? args.a_exp[tok] : 0;
      }
      __syncthreads();
      // The pass body is compiled for one and for two 16-row tiles, so that
      // only the rows in use are staged and every count below is a constant.
      auto body = [&](auto nt_tag) {
      constexpr int NT = decltype(nt_tag)::value;
      // Activation staging: NT*16 rows x 32 16-byte vectors per chunk; thread
      // -> row st_r, vectors v0 .. v0 + kVec - 1 (vector v = 4 g + j: group g,
      // subgroup j).
      constexpr int kVec = NT * 16 * 32 / kThreads;
      constexpr int kTPR = 32 / kVec;  // threads per row
      const int st_r = tid / kTPR, v0 = (tid % kTPR) * kVec;
      // Rows without a token read row 0: MFMA rows are independent and those
      // rows are never stored, so no branch (and no load-counter drain).
      const int my_tok = max(tok_lds[st_r], 0);
      const u32x4* a_src =
          reinterpret_cast<const u32x4*>(p.A + static_cast<int64_t>(my_tok) * K) + v0;

      // Every global load below is unconditional (indices clamped) so the
      // compiler keeps counting outstanding loads across the ring.
      auto load_a = [&](int chunk, u32x4* ar) {
        chunk = min(chunk, nchunks - 1);
#pragma unroll
        for (int i = 0; i < kVec; ++i) ar[i] = a_src[chunk * (kChunkK / 8) + i];
      };
      auto store_a = [&](int buf, const u32x4* ar) {
        // Both dequant forms emit the pair order (d, d + 4); stage A to match.
        // 16-byte piece (group g = st_g, subgroup j) of a row goes to dword
        //   RNE : (g >> 2) * 64 + j * 16 + (g & 3) * 4   (lane q reads group 4h+q)
        //   FAST: (g >> 2) * 64 + (g & 3) * 16 + j * 4   (lane q reads subgroup q)
        // so the 16-byte reads of one MFMA are 4 dwords apart across lane groups
        // and the 16 rows are 136 dwords apart: bank-conflict free.
        // FAST: the prepared activations are already in this order (group g at
        // dword 16 g, subgroup j at + 4 j) and are copied as they are.
        uint32_t* row = reinterpret_cast<uint32_t*>(&a_lds[buf][st_r * kV2Stride]);
#pragma unroll
        for (int i = 0; i < kVec; ++i) {
          const int g = (v0 + i) >> 2, j = (v0 + i) & 3;
          if constexpr (kFast) {
            *reinterpret_cast<u32x4*>(row + 4 * (v0 + i)) = ar[i];
          } else {
            uint32_t in[4] = {ar[i][0], ar[i][1], ar[i][2], ar[i][3]}, o[4];
            perm8(in, o);
            const int off = (g >> 2) * 64 + j * 16 + (g & 3) * 4;
            *reinterpret_cast<u32x4*>(row + off) = u32x4{o[0], o[1], o[2], o[3]};
          }
        }
      };
      auto load_w = [&](int chunk, u32x4 (&wr)[2][2]) {
        chunk = min(chunk, nchunks - 1);
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            wr[c][h] = *reinterpret_cast<const u32x4*>(wrow[c] + (chunk * kChunkGroups + 4 * h) * 4);
      };
      // this lane's 8 bytes of the scales of chunk `chunk` (8 groups per row)
      auto load_spiece = [&](int chunk) -> uint2 {
        return *reinterpret_cast<const uint2*>(sp_src + min(chunk, nchunks - 1) * 8);
      };
      // (index the __shared__ array directly: a pointer variable would turn
      // these into flat accesses, which also count as vector-memory loads)
      auto store_spiece = [&](int chunk, uint2 v) {
        *reinterpret_cast<uint2*>(
            &s_lds[wave][sp_row * kSStride + (chunk % kSSlots) * 8 + sp_half * 4]) = v;
      };

      f32x4 acc[2][2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};

      auto compute = [&](int buf, int chunk, const u32x4 (&wr)[2][2]) {
        // the chunk's 8 group scales of both column rows
        uint32_t sr[2][4];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(
              &s_lds[wave][(16 * c + c16) * kSStride + (chunk % kSSlots) * 8]);
#pragma unroll
          for (int i = 0; i < 4; ++i) sr[c][i] = v[i];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if constexpr (kFast) {
            u32x4 w[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) { w[c] = wr[c][h]; transpose4(w[c]); }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              f16x8 bfrag[2];
              float sc[2];
#pragma unroll
              for (int c = 0; c < 2; ++c) {
                bfrag[c] = __builtin_bit_cast(f16x8, unpack_f16(w[c][j], kNibMask, kNibMaskHi));
                const uint32_t sw = sr[c][(4 * h + j) >> 1];
                sc[c] = __uint_as_float(((4 * h + j) & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
              }
#pragma unroll
              for (int t = 0; t < 2; ++t) {
                if (t >= NT) break;
                const f16x8 afrag = *reinterpret_cast<const f16x8*>(
                    &a_lds[buf][(t * 16 + c16) * kV2Stride + 2 * (h * 64 + j * 16 + q * 4)]);
                const f32x4 d2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    afrag, negc, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                  const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag, bfrag[c], d2, 0, 0, 0);
#pragma unroll
                  for (int i = 0; i < 4; ++i) acc[t][c][i] = fmaf(sc[c], d[i], acc[t][c][i]);
                }
              }
            }
          } else {
            RneScale ks[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              // scale of group 4h + q: word 2h + (q >> 1), half q & 1
              const uint32_t lo = (q & 2) ? sr[c][2 * h + 1] : sr[c][2 * h];
              ks[c] = rne_scale(__uint_as_float((q & 1) ? (lo & 0xFFFF0000u) : (lo << 16)));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              bf16x8 bfrag[2];
#pragma unroll
              for (int c = 0; c < 2; ++c) bfrag[c] = dequant_rne(wr[c][h][j], ks[c], kNibMask, kNibMaskHi);
#pragma unroll
              for (int t = 0; t < 2; ++t) {
                if (t >= NT) break;
                const bf16x8 afrag = *reinterpret_cast<const bf16x8*>(
                    &a_lds[buf][(t * 16 + c16) * kV2Stride + 2 * (h * 64 + j * 16 + q * 4)]);
#pragma unroll
                for (int c = 0; c < 2; ++c)
                  acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, bfrag[c], acc[t][c], 0, 0, 0);
              }
            }
          }
        }
      };

      // Register ring slot r holds, after step c with c % 4 == r, the loads
      // issued at that step: activations of chunk c+4 and the scale piece of
      // chunk c+11 (weights: chunk c+3 in slot (c+3) % 4).
      struct Stage {
        u32x4 a[kVec];
        uint2 sp;
      };
      Stage r0, r1, r2, r3;
      u32x4 w0[2][2], w1[2][2], w2[2][2], w3[2][2];
      auto issue = [&](int c, Stage& st, u32x4 (&wn)[2][2]) {
        load_a(c + 4, st.a);
        st.sp = load_spiece(c + 11);
        load_w(c + 3, wn);
      };
      // Prologue: scales of chunks 0-7 and activations of chunk 0 in LDS, then
      // the loads of the three steps "before" step 0, in the loop's order, so
      // the load-counter wait at the loop head is the same on both paths.
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) store_spiece(ch, load_spiece(ch));
      load_a(0, r0.a);
      store_a(0, r0.a);
      __builtin_amdgcn_sched_barrier(0);
      issue(-3, r1, w0);
      __builtin_amdgcn_sched_barrier(0);
      issue(-2, r2, w1);
      __builtin_amdgcn_sched_barrier(0);
      issue(-1, r3, w2);
      __builtin_amdgcn_sched_barrier(0);
      // step c: A(c+1) -> LDS buffer (c+1)&1 (freed by compute(c-1)) and the
      // scale piece of chunk c+8 -> its ring slot (last read at step c-8), both
      // from ring slot (c+1) % 4; issue step c's loads into slot c % 4 and
      // W(c+3); compute chunk c. LDS operations of one wave execute in order,
      // so the other lanes' scale reads see the piece without a barrier.
      auto step = [&](int c, const u32x4 (&wc)[2][2], u32x4 (&wn)[2][2], const Stage& st,
                      Stage& ld) {
        __syncthreads();
        store_a((c + 1) & 1, st.a);
        store_spiece(c + 8, st.sp);
        issue(c, ld, wn);
        if (c < nchunks) compute(c & 1, c, wc);
      };
      for (int c = 0; c < nchunks; c += kRing) {
        step(c, w0, w3, r1, r0);
        step(c + 1, w1, w0, r2, r1);
        step(c + 2, w2, w1, r3, r2);
        step(c + 3, w3, w2, r0, r3);
      }

#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (t >= NT) break;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int slot = slot_lds[t * 16 + q * 4 + i];
          if (slot < 0) continue;
          const int ex = kFast ? exp_lds[t * 16 + q * 4 + i] : 0;
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int n = n_base + 16 * c + c16;
            const float v = kFast ? ldexpf(acc[t][c][i], ex) : acc[t][c][i];
            if (n < N) p.out[static_cast<int64_t>(slot) * N + n] = v;
          }
        }
      }
      };
      if (MAXNT == 2 && ntiles == 2)
        body(std::integral_constant<int, MAXNT>{});
      else
        body(std::integral_constant<int, 1>{});
    }
  }
}


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

// Token-slot block size the stream kernel consumes (one MFMA row tile).
int int4_block_size() { return 16; }

bool int4_use_stream(int a_dtype, int group_size, int64_t K) {
  return a_dtype == XK_DT_BF16 && group_size == 32 && K % 32 == 0 && K >= 32;
}

bool int4_prefill_ok(int a_dtype, int group_size, int64_t K, int64_t N, int64_t E);
bool int4_ksplit_ok(int64_t K, int64_t N, int64_t E, int64_t numel);
bool int4_rs_ok(int64_t M, int64_t K, int64_t N, int64_t E);
int rs_slices(int64_t K);
int launch_int4_rs(const void* A, int64_t M, int64_t K, const int32_t* packed,
                   const uint16_t* scale, int64_t E, int64_t N, int64_t numel, int64_t top_k,
                   const int32_t* sorted_ids, const int32_t* offsets, float* slot_out,
                   hipStream_t stream);
int launch_int4_prefill(const void* A, int64_t K, const int32_t* packed, const uint16_t* scale,
                        int64_t E, int64_t N, int64_t numel, int64_t top_k,
                        const int32_t* sorted_ids, const int32_t* offsets, float* slot_out,
                        hipStream_t stream);

// Routed rows per expert (on average) from which the tile kernel replaces the
// weight-streaming kernels.
constexpr int64_t kPrefillRowsPerExpert = 64;

// FAST-mode activation preparation (int4_decode.hip): scratch layout and launch.
int64_t int4_gemm_workspace_bytes(int64_t M, int64_t K);
Int4Prep int4_prep_layout(void* workspace, int64_t M, int64_t K);
int launch_int4_prep(const uint16_t* A, int64_t M, int64_t K, const Int4Prep& prep,
                     hipStream_t stream);
int launch_int4_ksplit(const Int4Prep& prep, int64_t K, const int32_t* packed,
                       const uint16_t* scale, int64_t E, int64_t N, int64_t numel, int64_t top_k,
                       const int32_t* sorted_ids, const int32_t* offsets, float* slot_out,
                       hipStream_t stream);

// The grouped-GEMM kernel a call runs, from its shapes and flags only (not
// from pointers), so that the number of partial planes is known before the
// call. Pointer alignment the chosen kernel needs is checked at launch.
enum class Int4Kernel { kSimple, kStreamV1, kStreamV2, kKsplit, kRs, kTile };

Int4Kernel int4_choose(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K, int a_dtype,
                       int group_size, int flags) {
  if (!int4_use_stream(a_dtype, group_size, K)) return Int4Kernel::kSimple;
  const int64_t numel = M * top_k;
  const bool tile_ok = int4_prefill_ok(a_dtype, group_size, K, N, E);
  const bool want_tile = (flags & XK_INT4_FORCE_TILE) ||
                         (numel >= kPrefillRowsPerExpert * E && !(flags & XK_INT4_FORCE_STREAM));
  if (tile_ok && want_tile && !(flags & XK_INT4_V1)) return Int4Kernel::kTile;
  if (K % 256 != 0 || (K / 32) % 8 != 0 || (flags & XK_INT4_V1)) return Int4Kernel::kStreamV1;
  if (flags & XK_INT4_FAST_DEQUANT)
    return (numel <= 16 * E && int4_ksplit_ok(K, N, E, numel) && !(flags & XK_INT4_V2))
               ? Int4Kernel::kKsplit
               : Int4Kernel::kStreamV2;
  if (!(flags & XK_INT4_V2) && int4_rs_ok(M, K, N, E)) return Int4Kernel::kRs;
  return Int4Kernel::kStreamV2;
}

// Number of fp32 partial planes [parts, M * top_k, N] the grouped GEMM
// writes: the K slices of the decode stream kernel, else one.
int int4_gemm_parts(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K, int a_dtype,
                    int group_size, int flags) {
  return int4_choose(M, top_k, E, N, K, a_dtype, group_size, flags) == Int4Kernel::kRs
             ? rs_slices(K)
             : 1;
}

int launch_int4_gemm(const void* A, int a_dtype, int64_t M, int64_t K, const int32_t* packed,
                     const uint16_t* scale, int64_t E, int64_t N, int group_size,
                     const int32_t* topk_ids, int64_t top_k, const int32_t* emap,
                     int num_global, const int32_t* sorted_ids, const int32_t* offsets,
                     float* slot_out, int flags, void* workspace, int64_t workspace_bytes,
                     hipStream_t stream) {
  XK_REQUIRE(a_dtype == XK_DT_BF16 || a_dtype == XK_DT_FP32, "int4: bad A dtype %d", a_dtype);
  XK_REQUIRE(M >= 0 && top_k >= 1 && E >= 1 && N >= 1 && K >= 8, "int4: bad sizes");
  XK_REQUIRE(K % 8 == 0, "int4: K=%lld not a multiple of 8", (long long)K);
  XK_REQUIRE(group_size > 0 && K % group_size == 0, "int4: group_size=%d does not divide K",
             group_size);
  XK_REQUIRE(E <= 65535 && N < (int64_t(1) << 30) && K < (int64_t(1) << 30), "int4: size limit");
  const int64_t numel = M * top_k;
  XK_REQUIRE(numel < (int64_t(1) << 30), "int4: M*top_k too large");
  if (numel == 0) return XK_OK;
  const Int4Kernel kern = int4_choose(M, top_k, E, N, K, a_dtype, group_size, flags);
  if (kern != Int4Kernel::kSimple) {
    XK_REQUIRE(sorted_ids && offsets, "int4: stream kernels need align outputs");
    XK_REQUIRE(reinterpret_cast<uintptr_t>(A) % 16 == 0, "int4: A must be 16-byte aligned");
  }
  if (kern == Int4Kernel::kTile || kern == Int4Kernel::kRs || kern == Int4Kernel::kKsplit ||
      kern == Int4Kernel::kStreamV2)
    XK_REQUIRE(reinterpret_cast<uintptr_t>(packed) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(scale) % 16 == 0,
               "int4: packed weights and scales must be 16-byte aligned");
  switch (kern) {
    case Int4Kernel::kTile:
      return launch_int4_prefill(A, K, packed, scale, E, N, numel, top_k, sorted_ids, offsets,
                                 slot_out, stream);
    case Int4Kernel::kRs:
      return launch_int4_rs(A, M, K, packed, scale, E, N, numel, top_k, sorted_ids, offsets,
                            slot_out, stream);
    case Int4Kernel::kKsplit:
    case Int4Kernel::kStreamV2: {
      StreamArgs a{static_cast<const uint16_t*>(A), reinterpret_cast<const uint32_t*>(packed),
                   scale, sorted_ids, offsets, slot_out, int(K), int(N), int(numel), int(top_k), 1};
      V2Args v2{a, int(E), nullptr};
      constexpr int kW = XK_INT4_STREAM_WAVES;
      const int64_t items = E * cdiv(N, kW * kColsPerWave);
      // Few routed rows per expert (decode): 16-row passes, which halves the
      // activation LDS; an expert with more rows takes several passes.
      const bool one_tile = numel <= 16 * E;
      const int per_cu = one_tile ? XK_INT4_STREAM_OCC : 2;
      const dim3 g2(static_cast<unsigned>(std::min<int64_t>(items, per_cu * device_cu_count())));
      const dim3 b2(kW * 64);
      if (flags & XK_INT4_FAST_DEQUANT) {
        const int64_t need = int4_gemm_workspace_bytes(M, K);
        if (workspace == nullptr || workspace_bytes < need)
          return set_error(XK_ERR_WORKSPACE, "int4 gemm: workspace %lld B < %lld B",
                           (long long)workspace_bytes, (long long)need);
        XK_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
                   "int4 gemm: workspace must be 256-byte aligned");
        const Int4Prep prep = int4_prep_layout(workspace, M, K);
        if (int rc = launch_int4_prep(static_cast<const uint16_t*>(A), M, K, prep, stream)) return rc;
        v2.s.A = prep.a16;
        v2.a_exp = prep.a_exp;
        if (kern == Int4Kernel::kKsplit)
          return launch_int4_ksplit(prep, K, packed, scale, E, N, numel, top_k, sorted_ids,
                                    offsets, slot_out, stream);
        if (one_tile)
          hipLaunchKernelGGL((int4_stream_v2<Int4Mode::kFast, kW, 1>), g2, b2, 0, stream, v2);
        else
          hipLaunchKernelGGL((int4_stream_v2<Int4Mode::kFast, kW, 2>), g2, b2, 0, stream, v2);
      } else {
        if (one_tile)
          hipLaunchKernelGGL((int4_stream_v2<Int4Mode::kRne, kW, 1>), g2, b2, 0, stream, v2);
        else
          hipLaunchKernelGGL((int4_stream_v2<Int4Mode::kRne, kW, 2>), g2, b2, 0, stream, v2);
      }
      XK_CHECK_LAUNCH("int4_stream_v2");
      return XK_OK;
    }
    case Int4Kernel::kStreamV1: {
      StreamArgs a{static_cast<const uint16_t*>(A), reinterpret_cast<const uint32_t*>(packed),
                   scale, sorted_ids, offsets, slot_out, int(K), int(N), int(numel), int(top_k),
                   int((K / 32) % 8 == 0 && reinterpret_cast<uintptr_t>(scale) % 16 == 0)};
      const dim3 grid(static_cast<unsigned>(cdiv(N, kColsPerWG)), static_cast<unsigned>(E));
      if (flags & XK_INT4_FAST_DEQUANT) {
        hipLaunchKernelGGL(int4_stream_gemm, grid, dim3(256), 0, stream, a);
        XK_CHECK_LAUNCH("int4_stream_gemm");
      } else {
        hipLaunchKernelGGL(int4_stream_gemm_rne, grid, dim3(256), 0, stream, a);
        XK_CHECK_LAUNCH("int4_stream_gemm_rne");
      }
      return XK_OK;
    }
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
