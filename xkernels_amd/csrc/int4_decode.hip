// INT4 W4A16 decode-regime grouped GEMM for gfx950 with K split across the
// waves of a workgroup: the FAST dequant of the reference's
// _fused_moe_int4_kernel (src/xkernels/ops/moe/triton/moe_int4_kernel.py:78-272),
// math of the oracle reference.py:22-70 with exact (n - 8) * s weights.
//
// Decode experts hold ~11 routed rows, so every packed byte feeds one 16-row
// MFMA tile and the kernel is a weight stream. Three rules shape it (each one
// measured on MI355X):
//   * every 128-byte weight line is read whole within one step: the L2 (4 MiB
//     per XCD) turns over in a few microseconds under the stream, so two
//     halves read an iteration apart are fetched from HBM twice;
//   * no workgroup barrier inside the k loop: a barrier per chunk makes every
//     wave wait for the slowest wave's loads;
//   * vector-memory loads return in issue order, so every load a step waits
//     for is issued before the loads it does not need yet.
// Structure:
//   * work unit = (16-row pass of one expert, 128 output columns); a
//     workgroup of 4 waves owns a unit and wave w contracts the k lines
//     [w L/4, (w+1) L/4) (line = 256 k = one 128-byte line per weight row) for
//     all 128 columns;
//   * step = (line, 16-column tile): lane (c, q) loads bytes 16q and 64 + 16q
//     of column c's line, a v_permlane32/16_swap transpose gives lane q word q
//     of each of the 8 groups, and one v_mfma_f32_16x16x32_f16 per group
//     contracts fp16 1024+n / 1024+16n nibbles (one v_and_or_b32 per pair)
//     against the prepared activations; the group scale multiplies the MFMA
//     result and two v_mfma_f32_16x16x4_f32 per step add the offset
//     correction (per-row group sums x scales);
//   * the weight ring holds one line of steps (8 steps x 2 KiB per wave); the
//     next line's activations (whole 128-byte row lines), row corrections and
//     the 128 columns' scales (16 bytes per lane, shared with ds_bpermute) are
//     loaded before the line's weights, activations staged into a
//     wave-private LDS buffer at the start of their line, so a wait for them
//     leaves a full line (16 KiB per wave, 128 KiB per CU) of weights in
//     flight, and the small operands cost few memory instructions (they cost
//     as much as the weights when fetched per step). Loads are buffer loads:
//     the unit's weight / scale bases are SGPR descriptors, each lane keeps
//     32-bit offsets, and tile / line offsets are uniform;
//   * the 4 partial 16 x 128 tiles of a unit are summed through LDS (two
//     barriers per unit) and stored as fp32 per-slot rows times 2^e_row.
#include <climits>

#include "int4_common.h"

namespace xk {

int device_cu_count();

namespace {

constexpr int kKsWaves = 4;                 // waves per workgroup = K slices
constexpr int kKsCols = 128;                // output columns per unit
constexpr int kKsTiles = kKsCols / 16;      // MFMA column tiles per unit
constexpr int kKsEBlocks = 4;               // expert offsets cached per lane (E <= 256)
constexpr int kKsRedStride = kKsCols + 4;   // fp32 per partial row in LDS (bank skew)
constexpr int kKsMaxUnits = 48;             // units per workgroup (row-id table in LDS)
constexpr int kKsPerCU = 2;                 // workgroups per CU (two waves per SIMD)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Workgroup barrier for LDS data only: waits for this wave's LDS operations,
// not for its outstanding global loads (the weight ring stays in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Activations for the FAST kernels: row m of A (bf16 [M, K]) becomes fp16
//   A16[m, k'] = a[m, k] * 2^-e_m  (x 1/16 at the positions that meet 1024 + 16n)
// with k' the unpack order a0 a4 a1 a5 a2 a6 a3 a7 inside every 8 k, and e_m
// chosen so that max_k |a[m, k]| * 2^-e_m lies in [2^14, 2^15): every bf16 value
// within 2^-31 of the row maximum converts exactly, nothing overflows, and the
// GEMM epilogue multiplies the row by 2^e_m (exact). A zero or non-finite
// maximum keeps e_m = 0 (non-finite values propagate as they would).
// corr[m, g] = -(1032 * sum of the 1024+n-position values + 1152 * sum of the
// 1024+16n-position values) of group g, so that sum_k a' * unpacked + corr =
// sum_k a * (n - 8) * 2^-e_m.
__global__ void __launch_bounds__(256) int4_prep_a(const uint16_t* __restrict__ A, int K,
                                                   Int4Prep prep) {
  __shared__ uint32_t red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(A + static_cast<int64_t>(m) * K);
  u32x4* dst = reinterpret_cast<u32x4*>(prep.a16 + static_cast<int64_t>(m) * K);
  const int nv = K >> 3;  // 8-k vectors; 4 per group
  uint32_t mx = 0;
  for (int v = tid; v < nv; v += 256) {
    const u32x4 x = src[v];
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = max(mx, max(x[i] & 0x7FFFu, (x[i] >> 16) & 0x7FFFu));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
    mx = max(mx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), o)));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = max(max(red[0], red[1]), max(red[2], red[3]));
  // bf16 exponent field of the maximum (subnormal maxima count as exponent -126)
  const int ebits = static_cast<int>(mx >> 7);
  const int e = (mx == 0 || ebits == 0xFF) ? 0 : max(ebits, 1) - 127 - 14;
  if (tid == 0) prep.a_exp[m] = e;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  // nv is a multiple of 4 (K % 32 == 0) and the 256-thread stride keeps each
  // group's four vectors in four consecutive lanes
  for (int v = tid; v < nv; v += 256) {
    const u32x4 x = src[v];
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = ldexpf(__uint_as_float(x[i] << 16), -e);
      f[2 * i + 1] = ldexpf(__uint_as_float(x[i] & 0xFFFF0000u), -e);
    }
    // (a0, a4) (a1/16, a5/16) (a2, a6) (a3/16, a7/16)
    u32x4 o;
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float sc = (d & 1) ? 0.0625f : 1.0f;
      const h2 hv = {static_cast<_Float16>(f[d] * sc), static_cast<_Float16>(f[d + 4] * sc)};
      o[d] = __builtin_bit_cast(uint32_t, hv);
      const float pair = static_cast<float>(hv[0]) + static_cast<float>(hv[1]);
      if (d & 1) hi += pair; else lo += pair;
    }
    dst[v] = o;
    float c = -(1032.0f * lo + 1152.0f * hi);
    c += __shfl_xor(c, 1);
    c += __shfl_xor(c, 2);
    if ((v & 3) == 0) prep.a_corr[static_cast<int64_t>(m) * (K >> 5) + (v >> 2)] = c;
  }
}

struct KsArgs {
  Int4Prep prep;
  const uint32_t* packed;  // [E, N, K/8]
  const uint16_t* scale;   // [E, N, K/32] bf16
  const int32_t* sorted_ids;
  const int32_t* offsets;  // [E+1] padded prefix in slots, multiples of 16
  float* out;              // [numel, N]
  int K, N, E, numel, top_k;
};

__global__ void __launch_bounds__(kKsWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
int4_decode_ksplit(KsArgs p) {
  __shared__ __attribute__((aligned(16))) float red[kKsWaves * 16 * kKsRedStride];
  // each wave's activations of the current line, MFMA operand order:
  // [group][lane][16 bytes]
  __shared__ __attribute__((aligned(16))) u32x4 a_lds[kKsWaves][8 * 64];
  __shared__ int tab_sid[kKsMaxUnits * 16];
  __shared__ int tab_exp[kKsMaxUnits * 16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, q = lane >> 4;
  const int K = p.K, N = p.N, G = K >> 5, KW = K >> 3;
  const int lw = (K >> 8) / kKsWaves;   // lines per wave: wave w takes lines w, w + 4, ...
  const int nb = N / kKsCols;
  const uint32_t kNibMask = in_vgpr(0x000F000Fu), kNibMaskHi = in_vgpr(0x00F000F0u);

  // Padded expert offsets, one per lane: block b holds offsets[64 b + lane + 1].
  int off1[kKsEBlocks];
#pragma unroll
  for (int b = 0; b < kKsEBlocks; ++b) {
    const int e = 64 * b + lane;
    off1[b] = e < p.E ? p.offsets[e + 1] : INT_MAX;
  }
  const int units = (p.offsets[p.E] >> 4) * nb;
  const int grid = gridDim.x;
  if (static_cast<int>(blockIdx.x) >= units) return;
  auto tok_of = [&](int sid) { return sid < p.numel ? sid / p.top_k : 0; };

  // Row ids and row exponents of every unit this workgroup runs, read once
  // into LDS so that the k loop issues no loads besides its own stream.
  // Unit u: pass u / nb (rows sorted_ids[16 (u / nb) ...]), columns u % nb.
  const int my_units = (units - static_cast<int>(blockIdx.x) + grid - 1) / grid;
  for (int x = tid; x < my_units * 16; x += kKsWaves * 64) {
    const int u = blockIdx.x + (x >> 4) * grid;
    const int sid = p.sorted_ids[16 * (u / nb) + (x & 15)];
    tab_sid[x] = sid;
    tab_exp[x] = p.prep.a_exp[tok_of(sid)];
  }
  __syncthreads();

  // Expert of pass pu: the number of experts whose padded range ends at or
  // before row 16 pu.
  auto expert_of = [&](int pu) {
    int e = 0;
#pragma unroll
    for (int b = 0; b < kKsEBlocks; ++b) e += __popcll(__ballot(off1[b] <= 16 * pu));
    return e;
  };

  // Buffer resources: the unit's weight and scale bases are wave-uniform
  // (SGPR descriptors), each lane keeps one 32-bit offset per stream, and the
  // tile / line offsets are uniform, so the ring needs no 64-bit addresses.
  // Line i of wave w is global line 4 i + w, so at any time the four waves
  // read adjacent 128-byte weight lines, adjacent activation bytes and the
  // same 128-byte scale line.
  const __amdgpu_buffer_rsrc_t rsrc_a =
      __builtin_amdgcn_make_buffer_rsrc(p.prep.a16, 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsrc_c =
      __builtin_amdgcn_make_buffer_rsrc(p.prep.a_corr, 0, 0x7FFFFFFF, 0x00020000);
  const int w_lane = (c16 * KW + 32 * wave + 4 * q) * 4;   // bytes; + 512 per line
  const int s_lane = (lane * G + 8 * wave) * 2;            // bytes (column lane); + 64 per line
  // Activations are fetched in whole 128-byte row lines (lane -> row lane / 8
  // or 8 + lane / 8, 16 bytes at 16 (lane % 8) of each 128 bytes) and stored
  // to LDS in MFMA operand order: piece j of row r -> [group j / 4][r + 16 (j % 4)].
  const int a_piece = 8 * (lane & 7);                      // halves within the 128-byte line
  u32x4* const a_st = &a_lds[wave][((lane & 7) >> 2) * 64 + (lane >> 3) + 16 * (lane & 3)];
  struct UnitRes {
    __amdgpu_buffer_rsrc_t w, s;  // this unit's weight rows and scale rows
    int a0, a1, c;                // lane's activation (rows lane/8, 8 + lane/8) / correction offsets
  };
  auto unit_res = [&](int i) {  // i-th unit of this workgroup (clamped)
    const int ii = min(i, my_units - 1);
    const int u = blockIdx.x + ii * grid;
    const int e = expert_of(u / nb);
    const int64_t col0 = static_cast<int64_t>(e) * N + (u % nb) * kKsCols;
    const int tok = tok_of(tab_sid[16 * ii + c16]);
    const int t0 = tok_of(tab_sid[16 * ii + (lane >> 3)]);
    const int t1 = tok_of(tab_sid[16 * ii + 8 + (lane >> 3)]);
    return UnitRes{
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(p.packed + col0 * KW), 0,
                                          kKsCols * KW * 4, 0x00020000),
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.scale + col0 * G), 0,
                                          kKsCols * G * 2, 0x00020000),
        (t0 * K + 256 * wave + a_piece) * 2, (t1 * K + 256 * wave + a_piece) * 2,
        (tok * G + 8 * wave + q) * 4};
  };

  // Per-line operand set (loaded one line ahead): activations (8 x 16 bytes,
  // staged into LDS at the start of their line), the row corrections of
  // groups q and 4 + q, and the 8 group scales of columns lane and lane + 64.
  struct LineSet {
    u32x4 a[8];
    float c[2];
    u32x4 s[2];
  };
  LineSet ls;
  const u32x4* al = &a_lds[wave][lane];
  u32x4 wr[kKsTiles][2];    // weight ring: one line of steps
  f32x4 acc[kKsTiles];
#pragma unroll
  for (int t = 0; t < kKsTiles; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  int ui = 0;   // unit index among this workgroup's units
  int il = 0;   // line of the current unit
  UnitRes rc = unit_res(0), rn = unit_res(1);

  // Loads of line `ln` of the current unit (ln >= lw: line ln - lw of the next).
  auto issue_set = [&](int ln, LineSet& st) {
    const bool nx = ln >= lw;
    const int i = nx ? ln - lw : ln;
    const UnitRes& u = nx ? rn : rc;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      st.a[2 * k] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, u.a0 + 128 * k, 2048 * i, 0);
      st.a[2 * k + 1] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, u.a1 + 128 * k, 2048 * i, 0);
    }
    st.c[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc_c, u.c, 128 * i, 0));
    st.c[1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc_c, u.c + 16, 128 * i, 0));
    st.s[0] = __builtin_amdgcn_raw_buffer_load_b128(u.s, s_lane, 64 * i, 0);
    st.s[1] = __builtin_amdgcn_raw_buffer_load_b128(u.s, s_lane + 64 * G * 2, 64 * i, 0);
  };
  // Step loads of tile t, line `ln`: this lane's 32 bytes of the column's
  // 128-byte weight line.
  auto issue_w = [&](int ln, int t) {
    const bool nx = ln >= lw;
    const int i = nx ? ln - lw : ln;
    const __amdgpu_buffer_rsrc_t rw = nx ? rn.w : rc.w;
    const int so = t * 16 * KW * 4 + 512 * i;
    wr[t][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_lane, so, 0);
    wr[t][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_lane + 64, so, 0);
  };

  // Prologue in the loop's issue order: set(line 0), then W(line 0); the loop
  // issues set(l + 1) and then, step by step, W(l + 1) while consuming line
  // l, so on both paths into the loop the wait for a line's set leaves that
  // line's weights in flight.
  issue_set(0, ls);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < kKsTiles; ++t) {
    issue_w(0, t);
    __builtin_amdgcn_sched_barrier(0);
  }

  auto line = [&]() {
    // this line's activations -> LDS (the wave's reads of the previous line
    // have completed: their values fed the MFMAs), corrections kept
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a_st[128 * k] = ls.a[2 * k];
      a_st[128 * k + 8] = ls.a[2 * k + 1];
    }
    const float cur_c0 = ls.c[0], cur_c1 = ls.c[1];
    const u32x4 cur_s0 = ls.s[0], cur_s1 = ls.s[1];
    // activations of the next line, issued before this line's weight loads so
    // that waiting for them never waits for those
    issue_set(il + 1, ls);
    // (the scheduler would otherwise move the ring loads, shortening the
    // distance each load has to arrive)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < kKsTiles; ++t) {
      u32x4 w0 = wr[t][0], w1 = wr[t][1];
      // the 8 group scales of column 16 t + c, held by lane (16 t + c) % 64
      u32x4 sv;
      const u32x4& ss = t < 4 ? cur_s0 : cur_s1;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sv[j] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * (16 * (t & 3) + c16), static_cast<int>(ss[j])));
      // scales of groups q and 4 + q (operands of the correction MFMAs)
      const uint32_t p0 = (q & 2) ? sv[1] : sv[0], p1 = (q & 2) ? sv[3] : sv[2];
      const float sq0 = __uint_as_float((q & 1) ? (p0 & 0xFFFF0000u) : (p0 << 16));
      const float sq1 = __uint_as_float((q & 1) ? (p1 & 0xFFFF0000u) : (p1 << 16));
      transpose4(w0);
      transpose4(w1);
      // Three phases, so that neither the LDS reads nor the MFMA results sit on
      // the critical path: operands of all 8 groups, then 8 independent MFMAs
      // (each result over its own unpacked operand), then the scaled sums.
      u32x4 af[8];
      f32x4 d[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        af[g] = al[64 * g];
        d[g] = __builtin_bit_cast(f32x4, unpack_f16(g < 4 ? w0[g] : w1[g - 4], kNibMask, kNibMaskHi));
      }
#pragma unroll
      for (int g = 0; g < 8; ++g)
        d[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, af[g]),
                                                      __builtin_bit_cast(f16x8, d[g]),
                                                      f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const uint32_t sw = sv[g >> 1];
        const float sg = __uint_as_float((g & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(sg, d[g][i], acc[t][i]);
      }
      // offset correction: acc[row][col] += sum_g corr[row][g] * s[col][g]
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur_c0, sq0, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur_c1, sq1, acc[t], 0, 0, 0);
      issue_w(il + 1, t);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (++il < lw) return;
    // ---- unit done: sum the K-slice partials, store, advance ----
    float* r = &red[wave * 16 * kKsRedStride];
#pragma unroll
    for (int t = 0; t < kKsTiles; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r[(4 * q + i) * kKsRedStride + 16 * t + c16] = acc[t][i];
        acc[t][i] = 0.f;
      }
    lds_barrier();
    {
      const int row = tid >> 4, c8 = (tid & 15) * 8;
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
      for (int w = 0; w < kKsWaves; ++w) {
        const float* src = &red[(w * 16 + row) * kKsRedStride + c8];
        s0 += *reinterpret_cast<const f32x4*>(src);
        s1 += *reinterpret_cast<const f32x4*>(src + 4);
      }
      const int slot = tab_sid[16 * ui + row];
      if (slot < p.numel) {
        const int ex = tab_exp[16 * ui + row];
#pragma unroll
        for (int i = 0; i < 4; ++i) { s0[i] = ldexpf(s0[i], ex); s1[i] = ldexpf(s1[i], ex); }
        const int u = blockIdx.x + ui * grid;
        float* dst = &p.out[static_cast<int64_t>(slot) * N + (u % nb) * kKsCols + c8];
        *reinterpret_cast<f32x4*>(dst) = s0;
        *reinterpret_cast<f32x4*>(dst + 4) = s1;
      }
    }
    lds_barrier();  // partials read before the next unit writes them
    il = 0;
    ++ui;
    rc = rn;
    rn = unit_res(ui + 1);
  };
  while (ui < my_units) line();
}

}  // namespace

int64_t int4_gemm_workspace_bytes(int64_t M, int64_t K) {
  const auto r = [](int64_t x) { return (x + 255) / 256 * 256; };
  return r(M * K * 2) + r(M * 4) + r(M * (K / 32) * 4);
}

Int4Prep int4_prep_layout(void* workspace, int64_t M, int64_t K) {
  const auto r = [](int64_t x) { return (x + 255) / 256 * 256; };
  char* b = static_cast<char*>(workspace);
  return Int4Prep{reinterpret_cast<uint16_t*>(b), reinterpret_cast<int32_t*>(b + r(M * K * 2)),
                  reinterpret_cast<float*>(b + r(M * K * 2) + r(M * 4))};
}

int launch_int4_prep(const uint16_t* A, int64_t M, int64_t K, const Int4Prep& prep,
                     hipStream_t stream) {
  hipLaunchKernelGGL(int4_prep_a, dim3(static_cast<unsigned>(M)), dim3(256), 0, stream, A,
                     int(K), prep);
  XK_CHECK_LAUNCH("int4_prep_a");
  return XK_OK;
}

// Shapes the K-split kernel takes; the unit count bound keeps its LDS row-id
// table (units = padded rows / 16 * N / 128 over one workgroup per CU).
bool int4_ksplit_ok(int64_t K, int64_t N, int64_t E, int64_t numel) {
  if (K % (kKsWaves * 256) != 0 || N % kKsCols != 0 || E > 64 * kKsEBlocks) return false;
  const int64_t max_pad = numel + E * 15;
  const int64_t units = max_pad / 16 * (N / kKsCols);
  return cdiv(units, int64_t(kKsPerCU) * device_cu_count()) <= kKsMaxUnits;
}

int launch_int4_ksplit(const Int4Prep& prep, int64_t K, const int32_t* packed,
                       const uint16_t* scale, int64_t E, int64_t N, int64_t numel, int64_t top_k,
                       const int32_t* sorted_ids, const int32_t* offsets, float* slot_out,
                       hipStream_t stream) {
  KsArgs a{prep, reinterpret_cast<const uint32_t*>(packed), scale, sorted_ids, offsets,
           slot_out, int(K), int(N), int(E), int(numel), int(top_k)};
  hipLaunchKernelGGL(int4_decode_ksplit, dim3(static_cast<unsigned>(kKsPerCU * device_cu_count())),
                     dim3(kKsWaves * 64), 0, stream, a);
  XK_CHECK_LAUNCH("int4_decode_ksplit");
  return XK_OK;
}

}  // namespace xk
