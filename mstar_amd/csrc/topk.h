// Softmax top-k: one token per wave (the decode routing launch and the
// fused router), or one token per 16-lane row (the grid-wide and
// single-workgroup routing paths).  Restates TopKRouter.forward
// (mstar/model/components/moe.py:131-139) from the logits on.
#pragma once
#include "common.h"

namespace mstar {

template <typename LT>
__device__ inline float load_logit(const LT* p, int64_t i);
template <>
__device__ inline float load_logit<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ inline float load_logit<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_bits_to_f32(p[i]);
}
// fp16 logits (a block run in half precision)
template <>
__device__ inline float load_logit<_Float16>(const _Float16* p, int64_t i) {
  return (float)p[i];
}

// Order-preserving map fp32 -> uint32 (larger float, larger key).
__device__ __forceinline__ uint32_t float_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inverse of float_key.
__device__ __forceinline__ float key_float(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Softmax top-k of one token by one wave (EPL = experts per lane,
// ceil(E / 64); expert e sits in lane e % 64, slot e / 64).
//
// Selection: k rounds of argmax over order-preserving integer keys of the
// logits (softmax is monotonic, so ranking logits ranks probabilities).
// Each round is a DPP max over the wave, then a ballot for the lowest
// expert index holding that key (ties go to the lower index), which is
// removed for the next round.  Ranks come out in order (value descending,
// ties by index).  The softmax max and sum are DPP reductions too; nothing
// goes through LDS.  emit(rank, expert, weight) runs on lane `rank` for
// each of the k selections (k <= 64).
template <int EPL, typename Emit>
__device__ __forceinline__ void topk_wave(const float (&v)[EPL], int E, int k, int renorm, int lane,
                                          const Emit& emit) {
  uint32_t key[EPL];
  float mxl = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const bool valid = j * 64 + lane < E;
    key[j] = valid ? float_key(v[j]) : 0u;  // 0 is below every valid key
    mxl = fmaxf(mxl, valid ? v[j] : -INFINITY);
  }
  const float mx = wave_fmax_dpp(mxl);
  float sl = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) sl += j * 64 + lane < E ? __expf(v[j] - mx) : 0.f;
  const float s = wave_fsum_dpp(sl);

  float my_p = 0.f, psum = 0.f;
  int my_id = 0;
  for (int r = 0; r < k; ++r) {
    uint32_t lm = key[0];
#pragma unroll
    for (int j = 1; j < EPL; ++j) lm = max(lm, key[j]);
    const uint32_t m = wave_umax_dpp(lm);
    int sel = -1;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const uint64_t b = __ballot(key[j] == m);
      if (sel < 0 && b) sel = j * 64 + __builtin_ctzll(b);
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (sel == j * 64 + lane) key[j] = 0u;
    const float p = __expf(key_float(m) - mx) / s;
    psum += p;
    if (lane == r) {
      my_p = p;
      my_id = sel;
    }
  }
  if (lane < k) emit(lane, my_id, renorm ? my_p / psum : my_p);
}

// Top-k of tokens t0, t0 + stride, ... (< t1) by one wave, a batch at a
// time: the logit rows of a batch are loaded together, so the wave waits
// for memory once per batch instead of once per token (batch size shrinks
// with the experts per lane to stay within 128 VGPRs).
// emit(token, rank, expert, weight).
template <typename LT, int EPL, typename Emit>
__device__ __forceinline__ void topk_tokens(const LT* __restrict__ logits, int64_t t0, int64_t t1,
                                            int64_t stride, int E, int k, int renorm, int lane,
                                            const Emit& emit) {
  constexpr int kTopkBatch = EPL >= 8 ? 1 : (EPL >= 4 ? 2 : 4);
  for (int64_t tb = t0; tb < t1; tb += kTopkBatch * stride) {
    float v[kTopkBatch][EPL];
#pragma unroll
    for (int b = 0; b < kTopkBatch; ++b) {
      const int64_t t = tb + b * stride;
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = j * 64 + lane;
        v[b][j] = (t < t1 && e < E) ? load_logit<LT>(logits + t * E, e) : -INFINITY;
      }
    }
#pragma unroll
    for (int b = 0; b < kTopkBatch; ++b) {
      const int64_t t = tb + b * stride;
      if (t >= t1) break;
      topk_wave<EPL>(v[b], E, k, renorm, lane,
                     [&](int r, int id, float w) { emit(t, r, id, w); });
    }
  }
}

// Minimum over a 16-lane row by DPP row rotations (every lane gets it).
__device__ __forceinline__ uint32_t row_umin16(uint32_t v) {
  v = min(v, (uint32_t)dpp_row_ror<1>((int)v));
  v = min(v, (uint32_t)dpp_row_ror<2>((int)v));
  v = min(v, (uint32_t)dpp_row_ror<4>((int)v));
  v = min(v, (uint32_t)dpp_row_ror<8>((int)v));
  return v;
}

// Softmax top-k of one token per 16-lane row (four tokens per wave), for
// E <= 16 * EPR and k <= 16: expert e in row lane e % 16, slot e / 16.
// The same selection as topk_wave -- k rounds of argmax over the
// order-preserving keys, ties to the lower expert index -- with row-wide
// DPP reductions, so a wave ranks four tokens at the instruction cost of
// about one.  The softmax sum is row lane 0's, broadcast to the row.
// emit(rank, expert, weight) runs on row lane `rank` (< k); `active` false
// rows (past the last token) take part in the reductions only.
template <int EPR, typename Emit>
__device__ __forceinline__ void topk_row16(const float (&v)[EPR], int E, int k, int renorm, int lane,
                                           bool active, const Emit& emit) {
  const int l16 = lane & 15;
  uint32_t key[EPR];
  float mxl = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPR; ++j) {
    const bool valid = j * 16 + l16 < E;
    key[j] = valid ? float_key(v[j]) : 0u;
    mxl = fmaxf(mxl, valid ? v[j] : -INFINITY);
  }
  const float mx = row_fmax16(mxl);
  float sl = 0.f;
#pragma unroll
  for (int j = 0; j < EPR; ++j) sl += j * 16 + l16 < E ? __expf(v[j] - mx) : 0.f;
  sl = row_fsum16(sl);  // row lane 0 holds the row's sum
  const float s = __shfl(sl, lane & ~15, 64);
  float my_p = 0.f, psum = 0.f;
  int my_id = 0;
  for (int r = 0; r < k; ++r) {
    uint32_t lm = key[0];
#pragma unroll
    for (int j = 1; j < EPR; ++j) lm = max(lm, key[j]);
    const uint32_t m = row_umax16(lm);
    uint32_t cand = 0xffffffffu;
#pragma unroll
    for (int j = EPR - 1; j >= 0; --j)
      if (key[j] == m) cand = (uint32_t)(j * 16 + l16);
    const int sel = (int)row_umin16(cand);
#pragma unroll
    for (int j = 0; j < EPR; ++j)
      if (sel == j * 16 + l16) key[j] = 0u;
    const float p = __expf(key_float(m) - mx) / s;
    psum += p;
    if (l16 == r) {
      my_p = p;
      my_id = sel;
    }
  }
  if (active && l16 < k) emit(l16, my_id, renorm ? my_p / psum : my_p);
}

// Top-k of tokens [tb, te) by the waves of a workgroup, four per wave at a
// time (one per 16-lane row): wave w takes tokens tb + 4 (w + nw n) + row.
// emit(token, rank, expert, weight).
template <typename LT, int EPR, typename Emit>
__device__ __forceinline__ void topk_tokens_rows(const LT* __restrict__ logits, int64_t tb, int64_t te, int w,
                                                 int nw, int E, int k, int renorm, int lane, const Emit& emit) {
  const int l16 = lane & 15, row = lane >> 4;
  for (int64_t base = tb + 4 * (int64_t)w; base < te; base += 4 * (int64_t)nw) {
    const int64_t t = base + row;
    const bool active = t < te;
    float v[EPR];
#pragma unroll
    for (int j = 0; j < EPR; ++j) {
      const int e = j * 16 + l16;
      v[j] = (active && e < E) ? load_logit<LT>(logits + t * E, e) : -INFINITY;
    }
    topk_row16<EPR>(v, E, k, renorm, lane, active, [&](int r, int id, float wt) { emit(t, r, id, wt); });
  }
}

}  // namespace mstar
