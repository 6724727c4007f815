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

namespace mstar {

template <typename LT>
__device__ inline float load_logit(const LT* p, int64_t i);
template <>
__device__ inline float load_logit<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ inline float load_logit<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_bits_to_f32(p[i]);
}

// EPL = experts per lane (ceil(E / 64)).
template <typename LT, int EPL>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const LT* __restrict__ logits,
                                                           int64_t M, int E, int k, int renorm,
                                                           float* __restrict__ w_out,
                                                           int32_t* __restrict__ ids32,
                                                           int64_t* __restrict__ ids64) {
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= M) return;
  const LT* row = logits + tok * E;
  float v[EPL];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    int e = j * 64 + lane;
    v[j] = e < E ? load_logit<LT>(row, e) : -INFINITY;
    mx = fmaxf(mx, v[j]);
  }
  mx = wave_max(mx);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    int e = j * 64 + lane;
    if (e < E) s += __expf(v[j] - mx);
  }
  s = wave_sum(s);
  unsigned taken = 0;  // bit j: v[j] already selected
  float sel_p = 0.f, psum = 0.f;
  int sel_id = 0;
  for (int t = 0; t < k; ++t) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      int e = j * 64 + lane;
      bool ok = e < E && !((taken >> j) & 1u);
      if (ok && (v[j] > bv || bi == 0x7fffffff)) { bv = v[j]; bi = e; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      float ov = __shfl_xor(bv, o, 64);
      int oi = __shfl_xor(bi, o, 64);
      bool take = (oi != 0x7fffffff) &&
                  (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi));
      if (take) { bv = ov; bi = oi; }
    }
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    float p = __expf(bv - mx) / s;
    psum += p;
    if (lane == t) { sel_p = p; sel_id = bi; }
  }
  if (lane < k) {
    float w = renorm ? sel_p / psum : sel_p;
    w_out[tok * k + lane] = w;
    if (ids32) ids32[tok * k + lane] = sel_id;
    if (ids64) ids64[tok * k + lane] = sel_id;
  }
}

// ---------------------------------------------------------------------------
// Alignment
// ---------------------------------------------------------------------------
constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kAlignBatch = 16;  // ids held per lane per batch

template <typename IT>
__device__ inline int load_expert(const IT* ids, int64_t i, int64_t end, int E) {
  if (i >= end) return E;
  int64_t e = (int64_t)ids[i];
  return (e < 0 || e >= E) ? E : (int)e;
}

// Lanes holding the same value as this lane (values in [0, 2^nbits)).
__device__ inline uint64_t match_any(int v, int nbits) {
  uint64_t m = ~0ull;
  for (int b = 0; b < nbits; ++b) {
    int bit = (v >> b) & 1;
    uint64_t bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  return m;
}

template <typename IT>
__global__ __launch_bounds__(kAlignThreads) void align_kernel(
    const IT* __restrict__ ids, int64_t numel, int E, int bm, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntpp, int64_t max_padded,
    int32_t* __restrict__ expert_off, int32_t* __restrict__ expert_cnt) {
  extern __shared__ int smem[];
  int* cnt = smem;                        // [kAlignWaves][E]: counts, then running bases
  int* off = cnt + kAlignWaves * E;       // [E + 1] padded exclusive offsets
  int* tot = off + E + 1;                 // [E] real counts
  int* wsum = tot + E;                    // [kAlignWaves] scan scratch
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nbits = 32 - __builtin_clz((unsigned)E);  // values 0..E

  for (int i = tid; i < kAlignWaves * E; i += kAlignThreads) cnt[i] = 0;
  __syncthreads();

  // Phase 1: per-wave histograms over contiguous chunks.
  const int64_t chunk = ((numel + kAlignWaves - 1) / kAlignWaves + 63) / 64 * 64;
  const int64_t c0 = (int64_t)w * chunk;
  const int64_t c1 = c0 + chunk < numel ? c0 + chunk : numel;
  int* mycnt = cnt + w * E;
  for (int64_t base = c0; base < c1; base += 64 * kAlignBatch) {
    int vals[kAlignBatch];
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) vals[r] = load_expert(ids, base + r * 64 + lane, c1, E);
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) {
      if (base + r * 64 >= c1) break;
      uint64_t m = match_any(vals[r], nbits);
      int leader = __builtin_ctzll(m);
      if (lane == leader && vals[r] < E) mycnt[vals[r]] += __builtin_popcountll(m);
    }
  }
  __syncthreads();

  // Phase 2: per expert, running bases across waves, padded counts, and an
  // exclusive block scan of the padded counts.
  int padded_local = 0;
  for (int e = tid; e < E; e += kAlignThreads) {
    int run = 0;
    for (int ww = 0; ww < kAlignWaves; ++ww) {
      int c = cnt[ww * E + e];
      cnt[ww * E + e] = run;
      run += c;
    }
    tot[e] = run;
    padded_local = (run + bm - 1) / bm * bm;  // E <= kAlignThreads: one expert per thread
  }
  int incl = wave_incl_scan(padded_local);
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  if (w == 0) {
    int ws = lane < kAlignWaves ? wsum[lane] : 0;
    int wi = wave_incl_scan(ws);
    if (lane < kAlignWaves) wsum[lane] = wi - ws;
  }
  __syncthreads();
  if (tid < E) off[tid] = wsum[w] + incl - padded_local;
  if (tid == E - 1) off[E] = wsum[w] + incl;
  __syncthreads();
  const int total_padded = off[E];
  if (tid == 0) *ntpp = total_padded;
  if (expert_off)
    for (int e = tid; e <= E; e += kAlignThreads) expert_off[e] = off[e];
  if (expert_cnt)
    for (int e = tid; e < E; e += kAlignThreads) expert_cnt[e] = tot[e];

  // Phase 3: expert_ids per block, padding positions, the tail.
  const int64_t max_blocks = (max_padded + bm - 1) / bm;
  for (int e = tid; e < E; e += kAlignThreads) {
    for (int i = off[e]; i < off[e + 1]; i += bm) expert_ids[i / bm] = e;
    for (int i = off[e] + tot[e]; i < off[e + 1]; ++i) sorted_ids[i] = (int32_t)numel;
  }
  for (int64_t i = total_padded / bm + tid; i < max_blocks; i += kAlignThreads) expert_ids[i] = 0;
  for (int64_t i = total_padded + tid; i < max_padded; i += kAlignThreads)
    sorted_ids[i] = (int32_t)numel;

  // Phase 4: stable scatter.  Within a wave, 64 consecutive slots per step;
  // lanes with equal experts are ranked by lane order, and the leader bumps
  // the wave's running base after everyone has read it.
  for (int64_t base = c0; base < c1; base += 64 * kAlignBatch) {
    int vals[kAlignBatch];
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) vals[r] = load_expert(ids, base + r * 64 + lane, c1, E);
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) {
      if (base + r * 64 >= c1) break;
      const int v = vals[r];
      uint64_t m = match_any(v, nbits);
      int rank = __builtin_popcountll(m & ((1ull << lane) - 1ull));
      int b = v < E ? mycnt[v] : 0;
      __builtin_amdgcn_wave_barrier();
      if (v < E) {
        sorted_ids[off[v] + b + rank] = (int32_t)(base + r * 64 + lane);
        if (rank == 0) mycnt[v] = b + __builtin_popcountll(m);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
int launch_topk_softmax(const void* logits, int logits_dtype, int64_t M, int E, int k,
                        int renorm, float* w, int32_t* ids32, int64_t* ids64,
                        hipStream_t stream) {
  if (M < 0 || E <= 0 || E > 1024 || k <= 0 || k > 64 || k > E || !w || (!ids32 && !ids64) ||
      (M > 0 && !logits)) {
    set_last_error("topk_softmax: invalid arguments (M=%lld E=%d k=%d)", (long long)M, E, k);
    return kInvalidArgument;
  }
  if (logits_dtype != kF32 && logits_dtype != kBF16) {
    set_last_error("topk_softmax: logits must be float32 or bfloat16");
    return kUnsupported;
  }
  if (M == 0) return kOk;
  dim3 grid((unsigned)((M + 3) / 4)), block(256);
  const int epl = (E + 63) / 64;
#define MSTAR_TOPK_CASE(N)                                                                   \
  case N:                                                                                    \
    if (logits_dtype == kF32)                                                                \
      topk_softmax_kernel<float, N><<<grid, block, 0, stream>>>((const float*)logits, M, E, \
                                                                k, renorm, w, ids32, ids64); \
    else                                                                                     \
      topk_softmax_kernel<uint16_t, N><<<grid, block, 0, stream>>>(                          \
          (const uint16_t*)logits, M, E, k, renorm, w, ids32, ids64);                        \
    break;
  switch (epl) {
    MSTAR_TOPK_CASE(1)
    MSTAR_TOPK_CASE(2)
    MSTAR_TOPK_CASE(4)
    MSTAR_TOPK_CASE(8)
    MSTAR_TOPK_CASE(16)
    default:
      if (epl == 3) {
        if (logits_dtype == kF32)
          topk_softmax_kernel<float, 4><<<grid, block, 0, stream>>>((const float*)logits, M, E, k,
                                                                   renorm, w, ids32, ids64);
        else
          topk_softmax_kernel<uint16_t, 4><<<grid, block, 0, stream>>>(
              (const uint16_t*)logits, M, E, k, renorm, w, ids32, ids64);
      } else if (epl <= 8) {
        if (logits_dtype == kF32)
          topk_softmax_kernel<float, 8><<<grid, block, 0, stream>>>((const float*)logits, M, E, k,
                                                                   renorm, w, ids32, ids64);
        else
          topk_softmax_kernel<uint16_t, 8><<<grid, block, 0, stream>>>(
              (const uint16_t*)logits, M, E, k, renorm, w, ids32, ids64);
      } else {
        if (logits_dtype == kF32)
          topk_softmax_kernel<float, 16><<<grid, block, 0, stream>>>(
              (const float*)logits, M, E, k, renorm, w, ids32, ids64);
        else
          topk_softmax_kernel<uint16_t, 16><<<grid, block, 0, stream>>>(
              (const uint16_t*)logits, M, E, k, renorm, w, ids32, ids64);
      }
  }
#undef MSTAR_TOPK_CASE
  return launch_status("topk_softmax");
}

int align_max_padded(int64_t numel, int E, int bm) { return (int)(numel + (int64_t)E * (bm - 1)); }

int launch_align(const void* ids, int ids_dtype, int64_t numel, int E, int bm,
                 int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp, int64_t max_padded,
                 int32_t* expert_off, int32_t* expert_cnt, hipStream_t stream) {
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
  if (ids_dtype != kI32 && ids_dtype != kI64) {
    set_last_error("moe_align_block_size: topk_ids must be int32 or int64");
    return kUnsupported;
  }
  size_t shmem = sizeof(int) * ((size_t)kAlignWaves * E + (E + 1) + E + kAlignWaves);
  static size_t attr_bytes = 0;  // LDS beyond 64 KB needs an explicit opt-in
  if (shmem > 64 * 1024 && shmem > attr_bytes) {
    if (hipFuncSetAttribute((const void*)align_kernel<int32_t>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem) != hipSuccess ||
        hipFuncSetAttribute((const void*)align_kernel<int64_t>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem) != hipSuccess) {
      set_last_error("moe_align_block_size: cannot reserve %zu bytes of LDS", shmem);
      return kLaunchError;
    }
    attr_bytes = shmem;
  }
  if (ids_dtype == kI32)
    align_kernel<int32_t><<<1, kAlignThreads, shmem, stream>>>(
        (const int32_t*)ids, numel, E, bm, sorted_ids, expert_ids, ntpp, max_padded, expert_off,
        expert_cnt);
  else
    align_kernel<int64_t><<<1, kAlignThreads, shmem, stream>>>(
        (const int64_t*)ids, numel, E, bm, sorted_ids, expert_ids, ntpp, max_padded, expert_off,
        expert_cnt);
  return launch_status("moe_align_block_size");
}

}  // namespace mstar
