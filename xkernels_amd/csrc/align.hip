// moe_align_block_size for gfx950.
//
// Semantics follow the reference oracle moe_align_block_size_ref
// (src/xkernels/ops/moe/w4a16.py:53-101): token-slots t = m*top_k + j are grouped
// by expert in ascending t (the stable argsort at w4a16.py:72), every expert's
// run is padded to a block_size multiple with pad id = numel, one expert id is
// emitted per block and unused trailing blocks read 0 (w4a16.py:91-96).
//
// Design (MI355X): counting sort from three steps that share device functions.
//   count   : LDS histogram of a contiguous slot chunk per workgroup (LDS atomics)
//   layout  : padded prefix over experts (wavefront shuffle scan), expert_ids by
//             binary search of the padded prefix, pad ids only into the gaps
//   scatter : stable in-chunk ranks from wavefront ballots. Lanes holding the
//             same expert find each other with one ballot per key bit; rank =
//             popcount(peers below me); waves are ordered through a small
//             per-wave LDS count table.
// Small problems run all three in ONE workgroup (one launch). Large ones launch
// a histogram grid, then one grid in which every workgroup re-derives the
// expert layout from the chunk histograms, scatters its chunk and writes its
// slice of expert_ids and pad ids (two launches, no single-workgroup phase).
#include <algorithm>

#include "common.h"

namespace xk {
namespace {

constexpr int kMaxExperts = 1024;  // local experts (after the EP remap)

__device__ __forceinline__ int key_bits(int num_experts) {
  // bits needed to hold keys 0..num_experts (num_experts = the "dropped" key)
  return 32 - __clz(num_experts);
}

// Block-wide exclusive scan of one int per thread (blockDim multiple of 64,
// at most 1024). `wsum` needs blockDim/64 ints of LDS. Returns the exclusive
// prefix; *total receives the block total.
__device__ int block_exclusive_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int s = lane < nw ? wsum[lane] : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      int y = __shfl_up(s, d, 64);
      if (lane >= d) s += y;
    }
    if (lane < nw) wsum[lane] = s;  // inclusive wave prefix
  }
  __syncthreads();
  int base = wave > 0 ? wsum[wave - 1] : 0;
  *total = wsum[nw - 1];
  __syncthreads();
  return base + x - v;
}

// LDS histogram of slots [begin, end) into cnt[0..num_experts).
__device__ void chunk_histogram(const int32_t* ids, int64_t begin, int64_t end,
                                const int32_t* emap, int num_global, int num_experts,
                                int* cnt) {
  for (int64_t t = begin + threadIdx.x; t < end; t += blockDim.x) {
    int e = map_expert(ids[t], emap, num_global, num_experts);
    if (e >= 0) atomicAdd(&cnt[e], 1);
  }
}

// Stable scatter of slots [begin, end): slot t of expert e goes to
// base[e] + (number of earlier slots of e in this chunk). base[] is advanced
// in place. wavecnt is [nwaves][num_experts+1] ints of LDS, zero on entry and
// zero again on exit; chunk_tot is [num_experts] ints of LDS scratch.
__device__ void chunk_stable_scatter(const int32_t* ids, int64_t begin, int64_t end,
                                     const int32_t* emap, int num_global, int num_experts,
                                     int* base, int* wavecnt, int* chunk_tot,
                                     int32_t* sorted_ids) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nbits = key_bits(num_experts);
  const int stride = num_experts + 1;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t c = begin; c < end; c += blockDim.x) {
    const int64_t t = c + threadIdx.x;
    int key = num_experts;
    if (t < end) {
      int e = map_expert(ids[t], emap, num_global, num_experts);
      if (e >= 0) key = e;
    }
    uint64_t peers = ~0ull;
    for (int b = 0; b < nbits; ++b) {
      const int bit = (key >> b) & 1;
      const uint64_t bal = __ballot(bit);
      peers &= bit ? bal : ~bal;
    }
    const int rank = __popcll(peers & below);
    const bool leader = rank == 0;
    if (leader && key < num_experts) wavecnt[wave * stride + key] = __popcll(peers);
    __syncthreads();
    if (key < num_experts) {
      int pos = base[key] + rank;
      for (int w = 0; w < wave; ++w) pos += wavecnt[w * stride + key];
      sorted_ids[pos] = static_cast<int32_t>(t);
    }
    const int nw = blockDim.x >> 6;
    for (int e = threadIdx.x; e < num_experts; e += blockDim.x) {
      int s = 0;
      for (int w = 0; w < nw; ++w) s += wavecnt[w * stride + e];
      chunk_tot[e] = s;
    }
    __syncthreads();
    if (leader && key < num_experts) wavecnt[wave * stride + key] = 0;
    for (int e = threadIdx.x; e < num_experts; e += blockDim.x) base[e] += chunk_tot[e];
    __syncthreads();
  }
}

// Given per-expert counts cnt[] (LDS), computes the padded exclusive prefix
// off[0..num_experts] (LDS), writes num_post, expert_offsets, expert_ids and
// the pad ids of every gap. Requires num_experts <= blockDim.x.
__device__ void emit_layout(const int* cnt, int* off, int* wsum, int num_experts,
                            int block_size, int64_t numel, int64_t max_pad,
                            int64_t max_blocks, int32_t* sorted_ids,
                            int32_t* expert_ids, int32_t* num_post,
                            int32_t* expert_offsets) {
  const int tid = threadIdx.x;
  int c = tid < num_experts ? cnt[tid] : 0;
  int padded = ((c + block_size - 1) / block_size) * block_size;
  int total = 0;
  int ex = block_exclusive_scan(padded, wsum, &total);
  if (tid < num_experts) off[tid] = ex;
  if (tid == 0) {
    off[num_experts] = total;
    num_post[0] = total;
  }
  __syncthreads();
  if (expert_offsets != nullptr)
    for (int e = tid; e <= num_experts; e += blockDim.x) expert_offsets[e] = off[e];
  // expert id of block b = #{e in [1, E] : off[e] <= b*bs}; blocks past total -> 0
  for (int64_t b = tid; b < max_blocks; b += blockDim.x) {
    const int64_t pos = b * block_size;
    int id = 0;
    if (pos < total) {
      int lo = 1, hi = num_experts;  // count of off[1..E] <= pos (off nondecreasing)
      while (lo <= hi) {
        int mid = (lo + hi) >> 1;
        if (off[mid] <= pos) lo = mid + 1; else hi = mid - 1;
      }
      id = lo - 1;
    }
    expert_ids[b] = id;
  }
  const int32_t pad = static_cast<int32_t>(numel);
  if (tid < num_experts)
    for (int p = ex + c; p < ex + padded; ++p) sorted_ids[p] = pad;
  for (int64_t p = total + tid; p < max_pad; p += blockDim.x) sorted_ids[p] = pad;
}

// ---------------------------------------------------------------- kernels ----

// Whole problem in one workgroup of 1024 threads.
__global__ void __launch_bounds__(1024)
align_single_wg(const int32_t* __restrict__ ids, int64_t numel, int num_experts,
                int block_size, const int32_t* __restrict__ emap, int num_global,
                int64_t max_pad, int64_t max_blocks, int32_t* __restrict__ sorted_ids,
                int32_t* __restrict__ expert_ids, int32_t* __restrict__ num_post,
                int32_t* __restrict__ expert_offsets) {
  extern __shared__ int lds[];
  const int nw = blockDim.x >> 6;
  int* cnt = lds;                               // [E]   histogram, then cursor
  int* off = cnt + num_experts;                 // [E+1] padded prefix
  int* tot = off + num_experts + 1;             // [E]   per-chunk totals
  int* wsum = tot + num_experts;                // [16]
  int* wavecnt = wsum + 16;                     // [nw][E+1]
  for (int i = threadIdx.x; i < num_experts; i += blockDim.x) cnt[i] = 0;
  for (int i = threadIdx.x; i < nw * (num_experts + 1); i += blockDim.x) wavecnt[i] = 0;
  __syncthreads();
  chunk_histogram(ids, 0, numel, emap, num_global, num_experts, cnt);
  __syncthreads();
  emit_layout(cnt, off, wsum, num_experts, block_size, numel, max_pad, max_blocks,
              sorted_ids, expert_ids, num_post, expert_offsets);
  __syncthreads();
  for (int i = threadIdx.x; i < num_experts; i += blockDim.x) cnt[i] = off[i];
  __syncthreads();
  chunk_stable_scatter(ids, 0, numel, emap, num_global, num_experts, cnt, wavecnt, tot,
                       sorted_ids);
}

// Grid phase 1: histogram of chunk b into chunk_cnt[b][0..E).
__global__ void __launch_bounds__(256)
align_count(const int32_t* __restrict__ ids, int64_t numel, int64_t chunk,
            int num_experts, const int32_t* __restrict__ emap, int num_global,
            int32_t* __restrict__ chunk_cnt) {
  extern __shared__ int lds[];
  for (int i = threadIdx.x; i < num_experts; i += blockDim.x) lds[i] = 0;
  __syncthreads();
  const int64_t begin = blockIdx.x * chunk;
  const int64_t end = min(numel, begin + chunk);
  chunk_histogram(ids, begin, end, emap, num_global, num_experts, lds);
  __syncthreads();
  for (int i = threadIdx.x; i < num_experts; i += blockDim.x)
    chunk_cnt[static_cast<int64_t>(blockIdx.x) * num_experts + i] = lds[i];
}

// Grid phase 2: every workgroup b of 1024 threads
//   * sums the chunk histograms column-wise: total count of every expert and
//     the count in chunks before b (independent loads, threads (expert, part));
//   * forms the padded expert prefix (block scan);
//   * stably scatters its own chunk;
//   * writes its 1/nchunks slice of expert_ids and of the pad ids (gap slots of
//     every expert and the tail), so the layout is written by the whole grid.
// Workgroup 0 also writes num_tokens_post_padded and expert_offsets.
__global__ void __launch_bounds__(1024)
align_place(const int32_t* __restrict__ ids, int64_t numel, int64_t chunk, int nchunks,
            int num_experts, int block_size, const int32_t* __restrict__ emap,
            int num_global, const int32_t* __restrict__ chunk_cnt, int64_t max_pad,
            int64_t max_blocks, int32_t* __restrict__ sorted_ids,
            int32_t* __restrict__ expert_ids, int32_t* __restrict__ num_post,
            int32_t* __restrict__ expert_offsets) {
  extern __shared__ int lds[];
  const int nw = blockDim.x >> 6;
  int* tot = lds;                          // [E]   total count of expert e
  int* base = tot + num_experts;           // [E]   count before this chunk, then cursor
  int* off = base + num_experts;           // [E+1] padded prefix
  int* wsum = off + num_experts + 1;       // [16]
  int* ctot = wsum + 16;                   // [E]   scatter scratch
  int* wavecnt = ctot + num_experts;       // [nw][E+1]
  int* part = wavecnt + nw * (num_experts + 1);  // [parts][2][E]
  const int b = blockIdx.x, tid = threadIdx.x;
  const int parts = max(1, static_cast<int>(blockDim.x) / num_experts);
  for (int i = tid; i < nw * (num_experts + 1); i += blockDim.x) wavecnt[i] = 0;
  {
    // thread (e, p): chunks [p*per, (p+1)*per) of expert e (for e < E when
    // E <= blockDim; otherwise one part and a loop over the experts)
    const int per = static_cast<int>(cdiv(nchunks, parts));
    for (int idx = tid; idx < parts * num_experts; idx += blockDim.x) {
      const int e = idx % num_experts, p = idx / num_experts;
      const int b0 = p * per, b1 = min(nchunks, b0 + per);
      int all = 0, before = 0;
      for (int c = b0; c < b1; ++c) {
        const int v = chunk_cnt[static_cast<int64_t>(c) * num_experts + e];
        all += v;
        before += c < b ? v : 0;
      }
      part[(2 * p) * num_experts + e] = all;
      part[(2 * p + 1) * num_experts + e] = before;
    }
  }
  __syncthreads();
  for (int e = tid; e < num_experts; e += blockDim.x) {
    int all = 0, before = 0;
    for (int p = 0; p < parts; ++p) {
      all += part[(2 * p) * num_experts + e];
      before += part[(2 * p + 1) * num_experts + e];
    }
    tot[e] = all;
    base[e] = before;
  }
  __syncthreads();
  // padded exclusive prefix over experts (num_experts <= blockDim)
  const int c = tid < num_experts ? tot[tid] : 0;
  const int padded = ((c + block_size - 1) / block_size) * block_size;
  int total = 0;
  const int ex = block_exclusive_scan(padded, wsum, &total);
  if (tid < num_experts) {
    off[tid] = ex;
    base[tid] += ex;
  }
  if (tid == 0) off[num_experts] = total;
  __syncthreads();
  if (b == 0) {
    if (tid == 0) num_post[0] = total;
    if (expert_offsets != nullptr)
      for (int e = tid; e <= num_experts; e += blockDim.x) expert_offsets[e] = off[e];
  }
  // this chunk's slots
  const int64_t begin = static_cast<int64_t>(b) * chunk;
  chunk_stable_scatter(ids, begin, min(numel, begin + chunk), emap, num_global, num_experts,
                       base, wavecnt, ctot, sorted_ids);
  // slice of the layout: expert of a position = #{e in [1, E] : off[e] <= pos}
  auto expert_at = [&](int64_t pos) {
    int lo = 1, hi = num_experts;
    while (lo <= hi) {
      const int mid = (lo + hi) >> 1;
      if (off[mid] <= pos) lo = mid + 1; else hi = mid - 1;
    }
    return lo - 1;
  };
  const int64_t bper = cdiv(max_blocks, nchunks);
  for (int64_t i = b * bper + tid; i < min(max_blocks, (b + 1) * bper); i += blockDim.x) {
    const int64_t pos = i * block_size;
    expert_ids[i] = pos < total ? expert_at(pos) : 0;
  }
  const int32_t pad = static_cast<int32_t>(numel);
  const int64_t sper = cdiv(max_pad, nchunks);
  for (int64_t sidx = b * sper + tid; sidx < min(max_pad, (b + 1) * sper); sidx += blockDim.x) {
    bool gap = sidx >= total;
    if (!gap) {
      const int e = expert_at(sidx);
      gap = sidx - off[e] >= tot[e];
    }
    if (gap) sorted_ids[sidx] = pad;
  }
}

constexpr int64_t kSingleWgMaxSlots = 8192;
constexpr int kSingleWgMaxExperts = 512;
constexpr int64_t kGridChunk = 1024;

bool use_single_wg(int64_t numel, int num_experts) {
  return numel <= kSingleWgMaxSlots && num_experts <= kSingleWgMaxExperts;
}

}  // namespace

// Bytes of scratch the grid path needs (0 when one workgroup suffices).
int64_t align_workspace_bytes(int64_t numel, int num_experts) {
  if (use_single_wg(numel, num_experts)) return 0;
  const int64_t nchunks = std::max<int64_t>(1, cdiv(numel, kGridChunk));
  return nchunks * num_experts * static_cast<int64_t>(sizeof(int32_t));
}

int launch_align(const int32_t* ids, int64_t numel, int num_experts, int block_size,
                 const int32_t* emap, int num_global, int32_t* sorted_ids,
                 int32_t* expert_ids, int32_t* num_post, int32_t* expert_offsets,
                 void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  XK_REQUIRE(num_experts > 0 && num_experts <= kMaxExperts,
             "align: num_experts=%d outside [1, %d]", num_experts, kMaxExperts);
  XK_REQUIRE(block_size > 0 && block_size <= 4096, "align: block_size=%d outside [1, 4096]",
             block_size);
  XK_REQUIRE(numel >= 0 && numel < (int64_t(1) << 30), "align: numel=%lld out of range",
             (long long)numel);
  XK_REQUIRE(sorted_ids && expert_ids && num_post, "align: null output pointer");
  XK_REQUIRE(numel == 0 || ids, "align: null topk_ids");
  XK_REQUIRE(emap == nullptr || num_global > 0, "align: expert_map needs num_global_experts > 0");
  const int64_t max_pad = numel + static_cast<int64_t>(num_experts + 1) * (block_size - 1);
  const int64_t max_blocks = cdiv(max_pad, block_size);
  if (use_single_wg(numel, num_experts)) {
    const int threads = 1024, nw = threads / 64;
    const size_t lds = sizeof(int) * (3 * num_experts + 1 + 16 + nw * (num_experts + 1));
    hipLaunchKernelGGL(align_single_wg, dim3(1), dim3(threads), lds, stream, ids, numel,
                       num_experts, block_size, emap, num_global, max_pad, max_blocks,
                       sorted_ids, expert_ids, num_post, expert_offsets);
    XK_CHECK_LAUNCH("align_single_wg");
    return XK_OK;
  }
  const int64_t need = align_workspace_bytes(numel, num_experts);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(XK_ERR_WORKSPACE, "align: workspace %lld B < %lld B",
                     (long long)workspace_bytes, (long long)need);
  const int nchunks = static_cast<int>(std::max<int64_t>(1, cdiv(numel, kGridChunk)));
  int32_t* chunk_cnt = static_cast<int32_t*>(workspace);
  hipLaunchKernelGGL(align_count, dim3(nchunks), dim3(256), sizeof(int) * num_experts,
                     stream, ids, numel, kGridChunk, num_experts, emap, num_global,
                     chunk_cnt);
  XK_CHECK_LAUNCH("align_count");
  {
    const int threads = 1024, nw = threads / 64;
    const int parts = std::max(1, threads / num_experts);
    const size_t lds = sizeof(int) * (4 * num_experts + 1 + 16 + nw * (num_experts + 1) +
                                      2 * parts * num_experts);
    hipLaunchKernelGGL(align_place, dim3(nchunks), dim3(threads), lds, stream, ids, numel,
                       kGridChunk, nchunks, num_experts, block_size, emap, num_global,
                       chunk_cnt, max_pad, max_blocks, sorted_ids, expert_ids, num_post,
                       expert_offsets);
    XK_CHECK_LAUNCH("align_place");
  }
  return XK_OK;
}

}  // namespace xk
