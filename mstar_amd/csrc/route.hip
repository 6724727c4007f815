// Routing and permutation kernels for gfx950.
//
//  * topk_softmax_kernel -- one wave64 per token: fp32 softmax statistics,
//    k rounds of a wave arg-max (ties -> lower expert index), optional
//    renormalisation.  Restates TopKRouter.forward
//    (mstar/model/components/moe.py:131-139) from the logits on.
//  * align_kernel -- the moe_align_block_size contract
//    (mstar/utils/fused_moe/align.py:55-103, csrc/moe_align_block_size.cu:
//    207-271) in ONE workgroup launch, with a deterministic order: within
//    an expert, slots are ascending (the stable argsort of align.py:146).
//    Sixteen waves each own a contiguous chunk of slots; per-(wave, expert)
//    counts live in LDS; a wave resolves equal experts among its 64 lanes
//    with a ballot-based match (no atomics), so the scatter is stable.
#include "common.h"
#include "launch.h"
#include "topk.h"

namespace mstar {


// One wave per token.  With `hidden`, a second wave per token quantises the
// token's bf16 hidden row per group of 128 for the FP8 expert GEMMs that
// follow (hq [M, H]: the e4m3fn values widened to bf16; hs [M, H/128]): the
// routing launch carries the activation quantisation.
template <typename LT, int EPL>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const LT* __restrict__ logits,
                                                           int64_t M, int E, int k, int renorm,
                                                           float* __restrict__ w_out,
                                                           int32_t* __restrict__ ids32,
                                                           int64_t* __restrict__ ids64,
                                                           const uint16_t* __restrict__ hidden,
                                                           int64_t H, uint16_t* __restrict__ hq,
                                                           float* __restrict__ hs, int* __restrict__ zero,
                                                           int n_zero) {
  const int lane = threadIdx.x & 63;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_zero; i += gridDim.x * blockDim.x) zero[i] = 0;
  // With `hidden`, two waves per token: the even one routes, the odd one
  // quantises the hidden row, in parallel.
  const int wpt = hidden ? 2 : 1;
  const int64_t gw = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t tok = gw / wpt;
  if (tok >= M) return;
  if (wpt == 2 && (gw & 1)) {
    constexpr int kQB = 4;  // groups of 128 per lane group in flight
    for (int64_t c0 = 0; c0 < H; c0 += kQB * 512) {
      v4i raw[kQB];
#pragma unroll
      for (int b = 0; b < kQB; ++b) {
        const int64_t c = c0 + (int64_t)b * 512 + lane * 8;
        raw[b] = c < H ? *(const v4i*)(hidden + tok * H + c) : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int b = 0; b < kQB; ++b) {
        const int64_t c = c0 + (int64_t)b * 512 + lane * 8;
        float sc;
        const int2 codes = quant_group8<kBF16>(raw[b], sc);
        if (c < H) {
          *(v4i*)(hq + tok * H + c) = fp8x8_to_bf16x8_bits(codes.x, codes.y);
          if ((lane & 15) == 0) hs[tok * (H / 128) + c / 128] = sc;
        }
      }
    }
    return;
  }
  float v[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * 64 + lane;
    v[j] = e < E ? load_logit<LT>(logits + tok * E, e) : -INFINITY;
  }
  topk_wave<EPL>(v, E, k, renorm, lane, [&](int r, int id, float w) {
    w_out[tok * k + r] = w;
    if (ids32) ids32[tok * k + r] = id;
    if (ids64) ids64[tok * k + r] = id;
  });
}

// ---------------------------------------------------------------------------
// Alignment building blocks (one 1024-thread workgroup = 16 waves)
// ---------------------------------------------------------------------------
constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kAlignBatch = 16;          // ids held per lane per batch
constexpr int kRouteSmallSlots = 4096;   // numel aligned by one workgroup
// Slots routed (top-k + alignment) by one workgroup.  Set with the
// one-token-per-wave top-k (about 500 VALU instructions per token), which
// made one CU the bottleneck beyond a few dozen tokens: 512 tokens took
// 115 us in one workgroup against 26 us over the grid-wide path (whose first
// pass also quantises the hidden rows).
constexpr int kRouteTopkSmallSlots = 512;
// Tokens per workgroup of the grid-wide routing: about 256 workgroups, 8 to
// 32 tokens each.  Fewer tokens per workgroup spread the top-k and the hidden
// quantisation over more CUs (512 tokens: 14 us at 8 per workgroup, 27 us at
// 32), but the scatter pass scans every earlier workgroup's histogram, so
// beyond about 256 workgroups it grows (8192 tokens at 8: 45 us of scatter).
static int route_tokens_per_block(int64_t M) {
  const int64_t t = (M + 255) / 256;
  return t < 8 ? 8 : t > 32 ? 32 : (int)t;
}

// Expert of slot i, or E for "skip" (out of range / beyond the end).
template <typename IT>
struct GlobalIds {
  const IT* ids;
  __device__ int operator()(int64_t i, int64_t end, int E) const {
    if (i >= end) return E;
    const int64_t e = (int64_t)ids[i];
    return (e < 0 || e >= E) ? E : (int)e;
  }
};
struct LdsIds {
  const int* ids;
  __device__ int operator()(int64_t i, int64_t end, int E) const {
    if (i >= end) return E;
    const int e = ids[i];
    return (e < 0 || e >= E) ? E : e;
  }
};

// Lanes holding the same value as this lane (values in [0, 2^nbits)).
__device__ __forceinline__ uint64_t match_any(int v, int nbits) {
  uint64_t m = ~0ull;
  for (int b = 0; b < nbits; ++b) {
    int bit = (v >> b) & 1;
    uint64_t bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  return m;
}

// Each wave owns a contiguous 64-aligned sub-range of [s0, s1).
__device__ __forceinline__ void wave_chunk(int64_t s0, int64_t s1, int w, int64_t& c0, int64_t& c1) {
  const int64_t n = s1 - s0;
  const int64_t chunk = ((n + kAlignWaves - 1) / kAlignWaves + 63) / 64 * 64;
  c0 = s0 + (int64_t)w * chunk;
  c1 = c0 + chunk < s1 ? c0 + chunk : s1;
  if (c0 > s1) c0 = s1;
}

// wcnt[w * E + e] = number of slots of expert e in wave w's sub-range.
// Leaders of equal-expert lane groups add the group size: no atomics.
template <typename Load>
__device__ __forceinline__ void range_counts(const Load& load, int64_t s0, int64_t s1, int E, int* wcnt) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nbits = 32 - __builtin_clz((unsigned)E);
  for (int i = tid; i < kAlignWaves * E; i += kAlignThreads) wcnt[i] = 0;
  __syncthreads();
  int64_t c0, c1;
  wave_chunk(s0, s1, w, c0, c1);
  int* mycnt = wcnt + w * E;
  for (int64_t base = c0; base < c1; base += 64 * kAlignBatch) {
    int vals[kAlignBatch];
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) vals[r] = load(base + r * 64 + lane, c1, E);
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) {
      if (base + r * 64 >= c1) break;
      const uint64_t m = match_any(vals[r], nbits);
      if (lane == __builtin_ctzll(m) && vals[r] < E) mycnt[vals[r]] += __builtin_popcountll(m);
    }
  }
  __syncthreads();
}

// Per expert: exclusive prefix of wcnt across waves (in place); tot[e] = sum.
__device__ __forceinline__ void range_wave_prefix(int* wcnt, int E, int* tot) {
  for (int e = threadIdx.x; e < E; e += kAlignThreads) {
    int run = 0;
    for (int ww = 0; ww < kAlignWaves; ++ww) {
      const int c = wcnt[ww * E + e];
      wcnt[ww * E + e] = run;
      run += c;
    }
    tot[e] = run;
  }
  __syncthreads();
}

// off[0..E] = exclusive scan of roundup(cnt[e], bm).  E < 1024: one expert
// per thread, wave scans plus a scan of the wave sums.
__device__ __forceinline__ void expert_scan(const int* cnt, int E, int bm, int* off, int* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int padded = tid < E ? (cnt[tid] + bm - 1) / bm * bm : 0;
  const int incl = wave_incl_scan(padded);
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  if (w == 0) {
    const int ws = lane < kAlignWaves ? wsum[lane] : 0;
    const int wi = wave_incl_scan(ws);
    if (lane < kAlignWaves) wsum[lane] = wi - ws;
  }
  __syncthreads();
  if (tid < E) off[tid] = wsum[w] + incl - padded;
  if (tid == E - 1) off[E] = wsum[w] + incl;
  __syncthreads();
}

// expert_ids of every block, padding slots, the tail, and the extras.
__device__ __forceinline__ void write_meta(const int* off, const int* tot, int E, int bm, int64_t numel,
                           int64_t max_padded, int32_t* sorted_ids, int32_t* expert_ids,
                           int32_t* ntpp, int32_t* expert_off, int32_t* expert_cnt) {
  const int tid = threadIdx.x;
  const int total_padded = off[E];
  if (tid == 0) *ntpp = total_padded;
  if (expert_off)
    for (int e = tid; e <= E; e += kAlignThreads) expert_off[e] = off[e];
  if (expert_cnt)
    for (int e = tid; e < E; e += kAlignThreads) expert_cnt[e] = tot[e];
  const int64_t max_blocks = (max_padded + bm - 1) / bm;
  for (int e = tid; e < E; e += kAlignThreads)
    for (int i = off[e]; i < off[e + 1]; i += bm) expert_ids[i / bm] = e;
  // Padding slots of each expert: a group of G threads per expert.
  const int G = E >= kAlignThreads ? 1 : kAlignThreads / E;
  for (int e = tid / G; e < E; e += kAlignThreads / G)
    for (int i = off[e] + tot[e] + tid % G; i < off[e + 1]; i += G) sorted_ids[i] = (int32_t)numel;
  for (int64_t i = total_padded / bm + tid; i < max_blocks; i += kAlignThreads) expert_ids[i] = 0;
  for (int64_t i = total_padded + tid; i < max_padded; i += kAlignThreads)
    sorted_ids[i] = (int32_t)numel;
}

// Stable scatter of [s0, s1): slot i of expert e goes to
// base[e] + (slots of e in earlier waves) + (earlier slots of e in this wave).
template <typename Load>
__device__ __forceinline__ void range_scatter(const Load& load, int64_t s0, int64_t s1, int E, const int* base,
                              int* wcnt, int32_t* sorted_ids) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nbits = 32 - __builtin_clz((unsigned)E);
  int64_t c0, c1;
  wave_chunk(s0, s1, w, c0, c1);
  int* mycnt = wcnt + w * E;
  for (int64_t b0 = c0; b0 < c1; b0 += 64 * kAlignBatch) {
    int vals[kAlignBatch];
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) vals[r] = load(b0 + r * 64 + lane, c1, E);
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) {
      if (b0 + r * 64 >= c1) break;
      const int v = vals[r];
      const uint64_t m = match_any(v, nbits);
      const int rank = __builtin_popcountll(m & ((1ull << lane) - 1ull));
      const int b = v < E ? mycnt[v] : 0;
      __builtin_amdgcn_wave_barrier();
      if (v < E) {
        sorted_ids[base[v] + b + rank] = (int32_t)(b0 + r * 64 + lane);
        if (rank == 0) mycnt[v] = b + __builtin_popcountll(m);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// LDS layout of the single-workgroup paths (ints): wcnt[16E] off[E+1] tot[E] wsum[16]
template <typename Load>
__device__ __forceinline__ void single_block_align(int* smem, int64_t numel, int E, int bm,
                                          int64_t max_padded, int32_t* sorted_ids,
                                          int32_t* expert_ids, int32_t* ntpp,
                                          int32_t* expert_off, int32_t* expert_cnt,
                                          const Load& load) {
  int* wcnt = smem;
  int* off = wcnt + kAlignWaves * E;
  int* tot = off + E + 1;
  int* wsum = tot + E;
  range_counts(load, 0, numel, E, wcnt);
  range_wave_prefix(wcnt, E, tot);
  expert_scan(tot, E, bm, off, wsum);
  write_meta(off, tot, E, bm, numel, max_padded, sorted_ids, expert_ids, ntpp, expert_off,
             expert_cnt);
  range_scatter(load, 0, numel, E, off, wcnt, sorted_ids);
}

// moe_align_block_size in one workgroup (numel <= kRouteSmallSlots, or no
// scratch for the grid-wide path).
template <typename IT>
__global__ __launch_bounds__(kAlignThreads) void align_kernel(
    const IT* __restrict__ ids, int64_t numel, int E, int bm, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntpp, int64_t max_padded,
    int32_t* __restrict__ expert_off, int32_t* __restrict__ expert_cnt) {
  extern __shared__ int smem[];
  single_block_align(smem, numel, E, bm, max_padded, sorted_ids, expert_ids, ntpp, expert_off,
                     expert_cnt, GlobalIds<IT>{ids});
}

// Softmax top-k of every token plus the alignment, in one workgroup: the
// decode-sized routing step is a single launch.
template <typename LT, int EPL>
__global__ __launch_bounds__(kAlignThreads) void route_small_kernel(
    const LT* __restrict__ logits, int64_t M, int E, int k, int renorm, float* __restrict__ w_out,
    int32_t* __restrict__ ids32, int64_t* __restrict__ ids64, int bm,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntpp,
    int64_t max_padded, int32_t* __restrict__ expert_off, int32_t* __restrict__ expert_cnt) {
  extern __shared__ int smem[];
  int* sIds = smem;                         // [M * k]
  int* rest = sIds + ((M * k + 3) & ~3ll);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const auto put = [&](int64_t t, int r, int id, float wt) {
    w_out[t * k + r] = wt;
    sIds[t * k + r] = id;
    if (ids32) ids32[t * k + r] = id;
    if (ids64) ids64[t * k + r] = id;
  };
  // Four tokens per wave (one per 16-lane row) when the experts fit a row.
  if (EPL <= 4 && k <= 16) topk_tokens_rows<LT, 4 * EPL>(logits, 0, M, w, kAlignWaves, E, k, renorm, lane, put);
  else topk_tokens<LT, EPL>(logits, w, M, kAlignWaves, E, k, renorm, lane, put);
  __syncthreads();
  single_block_align(rest, M * k, E, bm, max_padded, sorted_ids, expert_ids, ntpp, expert_off,
                     expert_cnt, LdsIds{sIds});
}

// ---- grid-wide path --------------------------------------------------------
// Pass 1 (top-k variant): top-k of `tpb` tokens per workgroup
// and the workgroup's expert histogram hist[b][E].  With `hidden` (bf16
// [M, H], H % 128 == 0) the workgroup also quantises its tokens' hidden rows
// per group of 128 into e4m3fn codes hq [M, H] and scales hs [M, H/128].
template <typename LT, int EPL>
__global__ __launch_bounds__(kAlignThreads) void topk_hist_kernel(
    const LT* __restrict__ logits, int64_t M, int E, int k, int renorm, float* __restrict__ w_out,
    int32_t* __restrict__ ids32, int64_t* __restrict__ ids64, int32_t* __restrict__ hist,
    const uint16_t* __restrict__ hidden, int64_t H, uint8_t* __restrict__ hq,
    float* __restrict__ hs, int tpb) {
  extern __shared__ int smem[];
  int* h = smem;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int e = threadIdx.x; e < E; e += kAlignThreads) h[e] = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)blockIdx.x * tpb;
  const int64_t t1 = t0 + tpb < M ? t0 + tpb : M;
  const auto put = [&](int64_t t, int r, int id, float wt) {
    w_out[t * k + r] = wt;
    ids32[t * k + r] = id;
    if (ids64) ids64[t * k + r] = id;
    atomicAdd(&h[id], 1);
  };
  if (EPL <= 4 && k <= 16) topk_tokens_rows<LT, 4 * EPL>(logits, t0, t1, w, kAlignWaves, E, k, renorm, lane, put);
  else topk_tokens<LT, EPL>(logits, t0 + w, t1, kAlignWaves, E, k, renorm, lane, put);
  if (hidden) {
    // 8-element chunks of the block's rows; 16 consecutive chunks (16
    // lanes) form one group of 128.
    constexpr int kQB = 4;
    const int64_t chunks = (t1 - t0) * (H / 8);
    const uint16_t* src = hidden + t0 * H;
    for (int64_t c0 = threadIdx.x; c0 < chunks; c0 += kQB * kAlignThreads) {
      v4i raw[kQB];
#pragma unroll
      for (int b = 0; b < kQB; ++b) {
        const int64_t c = c0 + (int64_t)b * kAlignThreads;
        raw[b] = c < chunks ? *(const v4i*)(src + c * 8) : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int b = 0; b < kQB; ++b) {
        const int64_t c = c0 + (int64_t)b * kAlignThreads;
        float sc;
        const int2 codes = quant_group8<kBF16>(raw[b], sc);
        if (c < chunks) {
          *(int2*)(hq + t0 * H + c * 8) = codes;
          if ((lane & 15) == 0) hs[t0 * (H / 128) + c / 16] = sc;
        }
      }
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kAlignThreads) hist[(int64_t)blockIdx.x * E + e] = h[e];
}

// Pass 1 (ids given): histogram of `per_block` slots per workgroup.
template <typename IT>
__global__ __launch_bounds__(kAlignThreads) void hist_kernel(const IT* __restrict__ ids,
                                                             int64_t numel, int E, int per_block,
                                                             int32_t* __restrict__ hist) {
  extern __shared__ int smem[];
  int* h = smem;
  for (int e = threadIdx.x; e < E; e += kAlignThreads) h[e] = 0;
  __syncthreads();
  const int64_t s0 = (int64_t)blockIdx.x * per_block;
  const GlobalIds<IT> load{ids};
  for (int64_t i = s0 + threadIdx.x; i < s0 + per_block && i < numel; i += kAlignThreads) {
    const int v = load(i, numel, E);
    if (v < E) atomicAdd(&h[v], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kAlignThreads) hist[(int64_t)blockIdx.x * E + e] = h[e];
}

// Pass 2: every workgroup rebuilds the expert offsets from hist (identical
// in all workgroups), workgroup 0 writes the metadata, and each workgroup
// scatters its own slots after the slots of the workgroups before it.
template <typename Load>
__global__ __launch_bounds__(kAlignThreads) void scatter_kernel(
    Load load, int64_t numel, int E, int bm, int per_block, int nblocks,
    const int32_t* __restrict__ hist, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntpp, int64_t max_padded,
    int32_t* __restrict__ expert_off, int32_t* __restrict__ expert_cnt) {
  extern __shared__ int smem[];
  int* wcnt = smem;                   // [16][E]
  int* off = wcnt + kAlignWaves * E;  // [E+1]
  int* tot = off + E + 1;             // [E]
  int* base = tot + E;                // [E]
  int* wsum = base + E;               // [16]
  const int b = blockIdx.x;
  {
    // Column sums of hist: `segs` threads per expert each add every
    // segs-th row (loads unrolled so they overlap), then one thread per
    // expert adds the partial sums.  wcnt holds the partials.
    const int segs = E * 8 <= kAlignThreads ? 8 : kAlignThreads / E;
    int* pall = wcnt;
    int* ppre = wcnt + segs * E;
    if (threadIdx.x < segs * E) {
      const int e = threadIdx.x % E, sg = threadIdx.x / E;
      int pre = 0, all = 0;
#pragma unroll 8
      for (int bb = sg; bb < nblocks; bb += segs) {
        const int c = hist[(int64_t)bb * E + e];
        pre += bb < b ? c : 0;
        all += c;
      }
      pall[sg * E + e] = all;
      ppre[sg * E + e] = pre;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kAlignThreads) {
      int pre = 0, all = 0;
      for (int sg = 0; sg < segs; ++sg) {
        all += pall[sg * E + e];
        pre += ppre[sg * E + e];
      }
      tot[e] = all;
      base[e] = pre;
    }
    __syncthreads();
  }
  expert_scan(tot, E, bm, off, wsum);
  if (b == 0)
    write_meta(off, tot, E, bm, numel, max_padded, sorted_ids, expert_ids, ntpp, expert_off,
               expert_cnt);
  for (int e = threadIdx.x; e < E; e += kAlignThreads) base[e] += off[e];
  const int64_t s0 = (int64_t)b * per_block;
  const int64_t s1 = s0 + per_block < numel ? s0 + per_block : numel;
  range_counts(load, s0, s1, E, wcnt);
  range_wave_prefix(wcnt, E, tot);
  range_scatter(load, s0, s1, E, base, wcnt, sorted_ids);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
int launch_topk_softmax(const void* logits, int logits_dtype, int64_t M, int E, int k,
                        int renorm, float* w, int32_t* ids32, int64_t* ids64,
                        hipStream_t stream, const void* hidden, int64_t H, uint16_t* hq,
                        float* hs, int* zero, int n_zero) {
  if (hidden && (H <= 0 || H % 512 != 0 || !hq || !hs)) {
    set_last_error("topk_softmax: hidden quantisation needs H %% 512 == 0 (H=%lld)", (long long)H);
    return kInvalidArgument;
  }
  if (M < 0 || E <= 0 || E > 1024 || k <= 0 || k > 64 || k > E ||
      (M > 0 && (!logits || !w || (!ids32 && !ids64)))) {
    set_last_error("topk_softmax: invalid arguments (M=%lld E=%d k=%d)", (long long)M, E, k);
    return kInvalidArgument;
  }
  if (logits_dtype != kF32 && logits_dtype != kBF16 && logits_dtype != kF16) {
    set_last_error("topk_softmax: logits must be float32, bfloat16 or float16");
    return kUnsupported;
  }
  if (M == 0) return kOk;
  // One wave per token.  Small batches get one-wave workgroups, so the
  // tokens spread over as many CUs as possible (the radix select is a long
  // dependent chain; one SIMD per token keeps it at issue latency).
  const int tpb = M <= 2048 ? 1 : 4;         // tokens per workgroup
  const int wpt = hidden ? 2 : 1;              // waves per token
  dim3 grid((unsigned)((M + tpb - 1) / tpb)), block(64 * tpb * wpt);
  const int epl = (E + 63) / 64;
#define MSTAR_TOPK_CASE(N)                                                                   \
  case N:                                                                                    \
    if (logits_dtype == kF32)                                                                \
      topk_softmax_kernel<float, N><<<grid, block, 0, stream>>>(                             \
          (const float*)logits, M, E, k, renorm, w, ids32, ids64, (const uint16_t*)hidden, H, \
          hq, hs, zero, n_zero);                                                        \
    else if (logits_dtype == kF16)                                                           \
      topk_softmax_kernel<_Float16, N><<<grid, block, 0, stream>>>(                          \
          (const _Float16*)logits, M, E, k, renorm, w, ids32, ids64, (const uint16_t*)hidden, \
          H, hq, hs, zero, n_zero);                                                     \
    else                                                                                     \
      topk_softmax_kernel<uint16_t, N><<<grid, block, 0, stream>>>(                          \
          (const uint16_t*)logits, M, E, k, renorm, w, ids32, ids64, (const uint16_t*)hidden, \
          H, hq, hs, zero, n_zero);                                                     \
    break;
  // Experts per lane, rounded up to a power of two (E <= 1024).
  const int epl2 = epl <= 1 ? 1 : epl <= 2 ? 2 : epl <= 4 ? 4 : epl <= 8 ? 8 : 16;
  switch (epl2) {
    MSTAR_TOPK_CASE(1)
    MSTAR_TOPK_CASE(2)
    MSTAR_TOPK_CASE(4)
    MSTAR_TOPK_CASE(8)
    MSTAR_TOPK_CASE(16)
  }
#undef MSTAR_TOPK_CASE
  return launch_status("topk_softmax");
}

int align_max_padded(int64_t numel, int E, int bm) { return (int)(numel + (int64_t)E * (bm - 1)); }

static size_t single_lds(int E) { return sizeof(int) * ((size_t)kAlignWaves * E + 2 * E + 1 + kAlignWaves); }
static size_t scatter_lds(int E) { return sizeof(int) * ((size_t)kAlignWaves * E + 3 * E + 1 + kAlignWaves); }

template <typename K>
static int opt_in_lds(K kern, size_t bytes) {
  return ensure_dynamic_lds((const void*)kern, bytes, "routing");
}

static int check_align_args(const void* ids, int64_t numel, int E, int bm, const int32_t* sorted_ids,
                            const int32_t* expert_ids, const int32_t* ntpp, int64_t max_padded) {
  // Mirrors the checks of moe_align_block_size (moe_align_block_size.cu:211-224):
  // the padded expert count must stay below 1024 (one scan thread per expert).
  const int64_t padded_e = ((int64_t)E + 31) / 32 * 32;
  if (E <= 0 || padded_e >= 1024) {
    set_last_error("moe_align_block_size: padded_num_experts must be less than 1024 (E=%d)", E);
    return kInvalidArgument;
  }
  if (bm <= 0 || numel < 0 || numel >= (int64_t)1 << 31 || !sorted_ids || !expert_ids || !ntpp ||
      (numel > 0 && !ids)) {
    set_last_error("moe_align_block_size: invalid arguments (numel=%lld bm=%d)",
                   (long long)numel, bm);
    return kInvalidArgument;
  }
  if (max_padded < numel + (int64_t)E * (bm - 1)) {
    set_last_error("moe_align_block_size: sorted_token_ids too small (%lld < %lld)",
                   (long long)max_padded, (long long)(numel + (int64_t)E * (bm - 1)));
    return kInvalidArgument;
  }
  return kOk;
}

size_t align_scratch_bytes(int64_t numel, int E) {
  const int64_t blocks = (numel + kAlignThreads - 1) / kAlignThreads;
  return (size_t)(blocks > 0 ? blocks : 1) * E * sizeof(int32_t);
}

bool route_is_grid(int64_t M, int k) { return M * k > kRouteTopkSmallSlots; }

size_t route_scratch_bytes(int64_t M, int k, int E) {
  const int tpb = route_tokens_per_block(M);
  const int64_t blocks = (M + tpb - 1) / tpb;
  return (size_t)(blocks > 0 ? blocks : 1) * E * sizeof(int32_t) + (size_t)M * k * sizeof(int32_t);
}

int launch_align(const void* ids, int ids_dtype, int64_t numel, int E, int bm,
                 int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp, int64_t max_padded,
                 int32_t* expert_off, int32_t* expert_cnt, void* scratch, size_t scratch_bytes,
                 hipStream_t stream) {
  int st = check_align_args(ids, numel, E, bm, sorted_ids, expert_ids, ntpp, max_padded);
  if (st != kOk) return st;
  if (ids_dtype != kI32 && ids_dtype != kI64) {
    set_last_error("moe_align_block_size: topk_ids must be int32 or int64");
    return kUnsupported;
  }
  const bool grid_path = numel > kRouteSmallSlots && scratch &&
                         scratch_bytes >= align_scratch_bytes(numel, E);
  if (!grid_path) {
    const size_t shmem = single_lds(E);
    if (ids_dtype == kI32) {
      if ((st = opt_in_lds(align_kernel<int32_t>, shmem)) != kOk) return st;
      align_kernel<int32_t><<<1, kAlignThreads, shmem, stream>>>(
          (const int32_t*)ids, numel, E, bm, sorted_ids, expert_ids, ntpp, max_padded, expert_off,
          expert_cnt);
    } else {
      if ((st = opt_in_lds(align_kernel<int64_t>, shmem)) != kOk) return st;
      align_kernel<int64_t><<<1, kAlignThreads, shmem, stream>>>(
          (const int64_t*)ids, numel, E, bm, sorted_ids, expert_ids, ntpp, max_padded, expert_off,
          expert_cnt);
    }
    return launch_status("moe_align_block_size");
  }
  const int nblocks = (int)((numel + kAlignThreads - 1) / kAlignThreads);
  int32_t* hist = (int32_t*)scratch;
  const size_t hshm = E * sizeof(int), sshm = scatter_lds(E);
  if (ids_dtype == kI32) {
    hist_kernel<int32_t><<<nblocks, kAlignThreads, hshm, stream>>>((const int32_t*)ids, numel, E,
                                                                   kAlignThreads, hist);
    if ((st = opt_in_lds(scatter_kernel<GlobalIds<int32_t>>, sshm)) != kOk) return st;
    scatter_kernel<<<nblocks, kAlignThreads, sshm, stream>>>(
        GlobalIds<int32_t>{(const int32_t*)ids}, numel, E, bm, kAlignThreads, nblocks, hist,
        sorted_ids, expert_ids, ntpp, max_padded, expert_off, expert_cnt);
  } else {
    hist_kernel<int64_t><<<nblocks, kAlignThreads, hshm, stream>>>((const int64_t*)ids, numel, E,
                                                                   kAlignThreads, hist);
    if ((st = opt_in_lds(scatter_kernel<GlobalIds<int64_t>>, sshm)) != kOk) return st;
    scatter_kernel<<<nblocks, kAlignThreads, sshm, stream>>>(
        GlobalIds<int64_t>{(const int64_t*)ids}, numel, E, bm, kAlignThreads, nblocks, hist,
        sorted_ids, expert_ids, ntpp, max_padded, expert_off, expert_cnt);
  }
  return launch_status("moe_align_block_size");
}

template <typename LT, int EPL>
static int route_impl(const void* logits, int64_t M, int E, int k, int renorm, float* w,
                      int32_t* ids32, int64_t* ids64, int bm, int32_t* sorted_ids,
                      int32_t* expert_ids, int32_t* ntpp, int64_t max_padded, int32_t* expert_off,
                      int32_t* expert_cnt, void* scratch, size_t scratch_bytes,
                      hipStream_t stream, const uint16_t* hidden, int64_t H, uint8_t* hq,
                      float* hs) {
  const int64_t numel = M * k;
  int st;
  if (numel <= kRouteTopkSmallSlots) {
    const size_t shmem = sizeof(int) * (size_t)((numel + 3) & ~3ll) + single_lds(E);
    if ((st = opt_in_lds(route_small_kernel<LT, EPL>, shmem)) != kOk) return st;
    route_small_kernel<LT, EPL><<<1, kAlignThreads, shmem, stream>>>(
        (const LT*)logits, M, E, k, renorm, w, ids32, ids64, bm, sorted_ids, expert_ids, ntpp,
        max_padded, expert_off, expert_cnt);
    return launch_status("moe_route");
  }
  if (!scratch || scratch_bytes < route_scratch_bytes(M, k, E)) {
    set_last_error("moe_route: scratch too small (%zu < %zu)", scratch_bytes,
                   route_scratch_bytes(M, k, E));
    return kWorkspaceTooSmall;
  }
  const int tpb = route_tokens_per_block(M);
  const int nblocks = (int)((M + tpb - 1) / tpb);
  int32_t* hist = (int32_t*)scratch;
  int32_t* tmp_ids = ids32 ? ids32 : hist + (size_t)nblocks * E;
  topk_hist_kernel<LT, EPL><<<nblocks, kAlignThreads, E * sizeof(int), stream>>>(
      (const LT*)logits, M, E, k, renorm, w, tmp_ids, ids64, hist, hidden, H, hq, hs, tpb);
  const size_t sshm = scatter_lds(E);
  if ((st = opt_in_lds(scatter_kernel<GlobalIds<int32_t>>, sshm)) != kOk) return st;
  scatter_kernel<<<nblocks, kAlignThreads, sshm, stream>>>(
      GlobalIds<int32_t>{tmp_ids}, numel, E, bm, tpb * k, nblocks, hist,
      sorted_ids, expert_ids, ntpp, max_padded, expert_off, expert_cnt);
  return launch_status("moe_route");
}

int launch_route(const void* logits, int logits_dtype, int64_t M, int E, int k, int renorm,
                 float* w, int32_t* ids32, int64_t* ids64, int bm, int32_t* sorted_ids,
                 int32_t* expert_ids, int32_t* ntpp, int64_t max_padded, int32_t* expert_off,
                 int32_t* expert_cnt, void* scratch, size_t scratch_bytes, hipStream_t stream,
                 const void* hidden, int64_t H, uint8_t* hq, float* hs) {
  if (M < 0 || k <= 0 || k > 64 || k > E || (M > 0 && (!logits || !w))) {
    set_last_error("moe_route: invalid arguments (M=%lld E=%d k=%d)", (long long)M, E, k);
    return kInvalidArgument;
  }
  int st = check_align_args(logits, M * k, E, bm, sorted_ids, expert_ids, ntpp, max_padded);
  if (st != kOk) return st;
  if (logits_dtype != kF32 && logits_dtype != kBF16 && logits_dtype != kF16) {
    set_last_error("moe_route: logits must be float32, bfloat16 or float16");
    return kUnsupported;
  }
  if (hidden && (!route_is_grid(M, k) || H <= 0 || H % 128 != 0 || !hq || !hs)) {
    set_last_error("moe_route: hidden-row quantisation needs the multi-workgroup path and "
                   "H %% 128 == 0 (M=%lld H=%lld)", (long long)M, (long long)H);
    return kInvalidArgument;
  }
  const uint16_t* hid = (const uint16_t*)hidden;
  const int epl = (E + 63) / 64;
#define MSTAR_ROUTE(N)                                                                          \
  return logits_dtype == kF32                                                                   \
             ? route_impl<float, N>(logits, M, E, k, renorm, w, ids32, ids64, bm, sorted_ids,   \
                                    expert_ids, ntpp, max_padded, expert_off, expert_cnt,       \
                                    scratch, scratch_bytes, stream, hid, H, hq, hs)             \
         : logits_dtype == kF16                                                                 \
             ? route_impl<_Float16, N>(logits, M, E, k, renorm, w, ids32, ids64, bm,            \
                                       sorted_ids, expert_ids, ntpp, max_padded, expert_off,    \
                                       expert_cnt, scratch, scratch_bytes, stream, hid, H, hq,  \
                                       hs)                                                      \
             : route_impl<uint16_t, N>(logits, M, E, k, renorm, w, ids32, ids64, bm,            \
                                       sorted_ids, expert_ids, ntpp, max_padded, expert_off,    \
                                       expert_cnt, scratch, scratch_bytes, stream, hid, H, hq,  \
                                       hs);
  if (epl <= 1) { MSTAR_ROUTE(1) }
  if (epl <= 2) { MSTAR_ROUTE(2) }
  if (epl <= 4) { MSTAR_ROUTE(4) }
  if (epl <= 8) { MSTAR_ROUTE(8) }
  MSTAR_ROUTE(16)
#undef MSTAR_ROUTE
}

}  // namespace mstar
