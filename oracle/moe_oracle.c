/*
 * moe_oracle.c — plain-C restatement of the xkernels quantized fused-MoE path.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (as the independent second oracle)
 * and by bench.py's CPU-baseline leg; never by the xkernels_amd package.
 *
 * Functions and the reference behaviour each follows (xkernels checkout):
 *   xko_align         src/xkernels/ops/moe/w4a16.py:53-101 (stable sort/pad),
 *                     EP drop of w4a16.py:104-155
 *   xko_dequant_int4  src/xkernels/ops/moe/w4a16.py:21-50
 *   xko_int4_moe      src/xkernels/ops/moe/reference.py:22-70
 *   xko_sum_reduce    src/xkernels/ops/moe/sum_reduce.py:20-39
 *   xko_dequant_mxfp4 src/xkernels/ops/gather/mxfp4.py:39-68
 *   xko_mxfp4_moe     src/xkernels/ops/moe/mxfp4_reference.py:28-112
 * Activations are passed as fp32 arrays holding the (bf16) values; `round_bf16`
 * flags reproduce the reference's bf16 roundings. OpenMP parallelises the
 * GEMM-shaped loops over output rows; each output is still a sequential fp32
 * sum over k.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Round-to-nearest-even fp32 -> bf16 -> fp32. */
static float bf16r(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u) { /* inf / nan: keep, quiet nan */
    if (u & 0x007FFFFFu) u |= 0x00400000u;
    u &= 0xFFFF0000u;
  } else {
    u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
  }
  memcpy(&f, &u, 4);
  return f;
}

float xko_bf16_round(float f) { return bf16r(f); }

static int map_expert(int id, const int32_t* emap, int nglobal, int nlocal) {
  if (emap) {
    if (id < 0 || id >= nglobal) return -1;
    id = emap[id];
  }
  return (id >= 0 && id < nlocal) ? id : -1;
}

/* Counting sort. sorted [numel + (E+1)(bs-1)], expert_ids [max_blocks] (tail 0). */
int xko_align(const int32_t* ids, int64_t numel, int E, int bs, const int32_t* emap, int nglobal,
              int32_t* sorted, int32_t* expert_ids, int64_t max_blocks, int32_t* num_post) {
  int64_t max_pad = numel + (int64_t)(E + 1) * (bs - 1);
  int64_t* cnt = calloc((size_t)E + 1, sizeof(int64_t));
  int64_t* off = calloc((size_t)E + 1, sizeof(int64_t));
  if (!cnt || !off) { free(cnt); free(off); return 1; }
  for (int64_t t = 0; t < numel; ++t) {
    int e = map_expert(ids[t], emap, nglobal, E);
    if (e >= 0) cnt[e]++;
  }
  for (int e = 0; e < E; ++e) off[e + 1] = off[e] + (cnt[e] + bs - 1) / bs * bs;
  for (int64_t p = 0; p < max_pad; ++p) sorted[p] = (int32_t)numel;
  for (int64_t b = 0; b < max_blocks; ++b) expert_ids[b] = 0;
  for (int e = 0; e < E; ++e)
    for (int64_t p = off[e]; p < off[e + 1]; p += bs) expert_ids[p / bs] = e;
  for (int e = 0; e < E; ++e) cnt[e] = off[e]; /* cursor */
  for (int64_t t = 0; t < numel; ++t) {    /* ascending t: stable */
    int e = map_expert(ids[t], emap, nglobal, E);
    if (e >= 0) sorted[cnt[e]++] = (int32_t)t;
  }
  *num_post = (int32_t)off[E];
  free(cnt);
  free(off);
  return 0;
}

/* rows of packed int4 [rows, K/8] with bf16 scales [rows, K/gs] -> fp32 [rows, K]. */
void xko_dequant_int4(const int32_t* packed, const uint16_t* scale, int64_t rows, int64_t K,
                      int gs, int round_bf16, float* out) {
  const int64_t G = K / gs;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t k = 0; k < K; ++k) {
      uint32_t w = (uint32_t)packed[r * (K / 8) + k / 8];
      int nib = (int)((w >> (4 * (k % 8))) & 0xFu);
      uint32_t sb = (uint32_t)scale[r * G + k / gs] << 16;
      float s;
      memcpy(&s, &sb, 4);
      float v = (float)(nib - 8) * s;
      out[r * K + k] = round_bf16 ? bf16r(v) : v;
    }
  }
}

/* out[M, N] fp32 = sum_j [w] * A[m] . W[e_j]^T ; A fp32 [M, K] holding its values. */
void xko_int4_moe(const float* A, int round_bf16, int64_t M, int64_t K, const int32_t* packed,
                  const uint16_t* scale, int64_t E, int64_t N, int gs, const int32_t* ids,
                  const float* w, int64_t top_k, const int32_t* emap, int nglobal, int mulw,
                  float* out) {
  const int64_t numel = M * top_k;
  memset(out, 0, sizeof(float) * (size_t)(M * N));
  /* per-slot contribution rows, summed in slot order per token afterwards */
  float* rows = calloc((size_t)(numel * N), sizeof(float));
  int* used = calloc((size_t)E, sizeof(int));
  if (!rows || !used) { free(rows); free(used); return; }
  for (int64_t t = 0; t < numel; ++t) {
    int e = map_expert(ids[t], emap, nglobal, (int)E);
    if (e >= 0) used[e] = 1;
  }
#pragma omp parallel
  {
    float* wrow = malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(dynamic, 16)
    for (int64_t en = 0; en < E * N; ++en) {
      const int64_t e = en / N, n = en % N;
      if (!used[e]) continue;
      xko_dequant_int4(packed + en * (K / 8), scale + en * (K / gs), 1, K, gs, round_bf16, wrow);
      for (int64_t t = 0; t < numel; ++t) {
        if (map_expert(ids[t], emap, nglobal, (int)E) != e) continue;
        const float* a = A + (t / top_k) * K;
        float acc = 0.f;
        for (int64_t k = 0; k < K; ++k) acc += a[k] * wrow[k];
        rows[t * N + n] = acc;
      }
    }
    free(wrow);
  }
  for (int64_t t = 0; t < numel; ++t) {
    if (map_expert(ids[t], emap, nglobal, (int)E) < 0) continue;
    const float f = mulw ? w[t] : 1.f;
    for (int64_t n = 0; n < N; ++n) out[(t / top_k) * N + n] += f * rows[t * N + n];
  }
  free(rows);
  free(used);
}

/* out[M, H] = s * sum_k w[m,k] * y[m,k,:] (w may be NULL). */
void xko_sum_reduce(const float* y, int64_t M, int64_t top_k, int64_t H, const float* w, float s,
                    float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t h = 0; h < H; ++h) {
      float acc = 0.f;
      for (int64_t k = 0; k < top_k; ++k)
        acc += y[(m * top_k + k) * H + h] * (w ? w[m * top_k + k] : 1.f);
      out[m * H + h] = acc * s;
    }
}

static const float kE2M1[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f,
                                -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};

/* rows of e2m1 pairs [rows, K/2] with e8m0 scales [rows, K/32] -> fp32 [rows, K]. */
void xko_dequant_mxfp4(const uint8_t* packed, const uint8_t* scale, int64_t rows, int64_t K,
                       float* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t k = 0; k < K; ++k) {
      uint8_t b = packed[r * (K / 2) + k / 2];
      int code = (k & 1) ? (b >> 4) : (b & 0xF);
      uint8_t sb = scale[r * (K / 32) + k / 32];
      float m = (sb == 0xFF) ? 0.f : ldexpf(1.f, (int)sb - 127);
      out[r * K + k] = kE2M1[code] * m;
    }
}

static float silu(float x) { return x / (1.f + expf(-x)); }

/* out[M, hidden] fp32 = sum_j [w] * (swiglu(bf16 A @ W13^T (+b13)) @ W2^T (+b2)). */
void xko_mxfp4_moe(const float* A, int64_t M, int64_t hidden, const uint8_t* w13,
                   const uint8_t* w13s, const uint8_t* w2, const uint8_t* w2s, int64_t E,
                   int64_t ispp, const float* b13, const float* b2, float limit,
                   const int32_t* ids, const float* w, int64_t top_k, const int32_t* emap,
                   int nglobal, int mulw, float* out) {
  const int64_t numel = M * top_k;
  memset(out, 0, sizeof(float) * (size_t)(M * hidden));
  float* act = calloc((size_t)(numel * ispp), sizeof(float));
  float* rows = calloc((size_t)(numel * hidden), sizeof(float));
  int* used = calloc((size_t)E, sizeof(int));
  if (!act || !rows || !used) { free(act); free(rows); free(used); return; }
  for (int64_t t = 0; t < numel; ++t) {
    int e = map_expert(ids[t], emap, nglobal, (int)E);
    if (e >= 0) used[e] = 1;
  }
#pragma omp parallel
  {
    float* wr = malloc(sizeof(float) * (size_t)(2 * hidden > ispp ? 2 * hidden : ispp));
#pragma omp for schedule(dynamic, 4)
    for (int64_t ej = 0; ej < E * ispp; ++ej) { /* stage 0: gate row j and up row ispp+j */
      const int64_t e = ej / ispp, j = ej % ispp;
      if (!used[e]) continue;
      xko_dequant_mxfp4(w13 + (e * 2 * ispp + j) * (hidden / 2), w13s + (e * 2 * ispp + j) * (hidden / 32), 1, hidden, wr);
      xko_dequant_mxfp4(w13 + (e * 2 * ispp + ispp + j) * (hidden / 2), w13s + (e * 2 * ispp + ispp + j) * (hidden / 32), 1, hidden, wr + hidden);
      for (int64_t t = 0; t < numel; ++t) {
        if (map_expert(ids[t], emap, nglobal, (int)E) != e) continue;
        const float* a = A + (t / top_k) * hidden;
        float g = 0.f, u = 0.f;
        for (int64_t k = 0; k < hidden; ++k) {
          const float x = bf16r(a[k]);
          g += x * bf16r(wr[k]);
          u += x * bf16r(wr[hidden + k]);
        }
        g = bf16r(g);
        u = bf16r(u);
        if (b13) {
          g = bf16r(g + b13[e * 2 * ispp + j]);
          u = bf16r(u + b13[e * 2 * ispp + ispp + j]);
        }
        if (limit > 0.f) {
          g = fminf(g, limit);
          u = fminf(fmaxf(u, -limit), limit);
        }
        act[t * ispp + j] = bf16r(silu(g) * u);
      }
    }
#pragma omp for schedule(dynamic, 16)
    for (int64_t en = 0; en < E * hidden; ++en) { /* stage 1: down row n */
      const int64_t e = en / hidden, n = en % hidden;
      if (!used[e]) continue;
      xko_dequant_mxfp4(w2 + en * (ispp / 2), w2s + en * (ispp / 32), 1, ispp, wr);
      for (int64_t t = 0; t < numel; ++t) {
        if (map_expert(ids[t], emap, nglobal, (int)E) != e) continue;
        float d = 0.f;
        for (int64_t k = 0; k < ispp; ++k) d += act[t * ispp + k] * bf16r(wr[k]);
        d = bf16r(d);
        if (b2) d = bf16r(d + b2[en]);
        rows[t * hidden + n] = d;
      }
    }
    free(wr);
  }
  for (int64_t t = 0; t < numel; ++t) {
    if (map_expert(ids[t], emap, nglobal, (int)E) < 0) continue;
    const float f = mulw ? w[t] : 1.f;
    for (int64_t n = 0; n < hidden; ++n) out[(t / top_k) * hidden + n] += f * rows[t * hidden + n];
  }
  free(act);
  free(rows);
  free(used);
}
