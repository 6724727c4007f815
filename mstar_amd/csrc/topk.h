// Softmax top-k of one token per wave: shared by the routing kernels and
// the decode gate_up kernel that routes in its prologue.  Restates
// TopKRouter.forward (mstar/model/components/moe.py:131-139) from the
// logits on.
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

// Softmax top-k (k <= 8) of four tokens per wave, one 16-lane row each, for
// E <= 128 experts: expert j + 16 i sits in lane j of the token's row,
// register i.  Keys are 64-bit -- the order-preserving logit key above the
// complement of the expert index -- so one descending order is "logit
// descending, lower index first", the order of topk_wave.  Each lane sorts
// its 8 keys (a 19-comparator network), then four merge rounds combine
// sorted lists of partner lanes (quad swaps, then rotations of the row by 4
// and 8 lanes), each keeping the top 8 of 16 with a half-cleaner and a
// bitonic merge; after them every lane of the row holds the row's top 8.
// The softmax statistics are row reductions.  emit(token, rank, expert,
// weight) runs on lane `rank` of each row with a token (tok >= 0).
struct TopkKey {
  uint64_t k;
};
__device__ __forceinline__ void topk_cas(uint64_t& a, uint64_t& b) {  // a <- max, b <- min
  const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
  a = hi;
  b = lo;
}
template <int CTRL>
__device__ __forceinline__ uint64_t topk_dpp64(uint64_t v) {
  const int lo = __builtin_amdgcn_update_dpp((int)(uint32_t)v, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp((int)(uint32_t)(v >> 32), (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}
template <int CTRL>
__device__ __forceinline__ void topk_merge_round(uint64_t (&key)[8]) {
  uint64_t other[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) other[i] = topk_dpp64<CTRL>(key[i]);
#pragma unroll
  for (int i = 0; i < 8; ++i) key[i] = key[i] > other[7 - i] ? key[i] : other[7 - i];
  topk_cas(key[0], key[4]); topk_cas(key[1], key[5]); topk_cas(key[2], key[6]); topk_cas(key[3], key[7]);
  topk_cas(key[0], key[2]); topk_cas(key[1], key[3]); topk_cas(key[4], key[6]); topk_cas(key[5], key[7]);
  topk_cas(key[0], key[1]); topk_cas(key[2], key[3]); topk_cas(key[4], key[5]); topk_cas(key[6], key[7]);
}

template <typename LT, typename Emit>
__device__ __forceinline__ void topk_rows16(const LT* __restrict__ logits, int64_t tok, int E, int k,
                                            int renorm, int lane, const Emit& emit) {
  const int j = lane & 15;
  float v[8];
  uint64_t key[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = j + 16 * i;
    const bool valid = tok >= 0 && e < E;
    v[i] = valid ? load_logit<LT>(logits + tok * E, e) : -INFINITY;
    key[i] = valid ? ((uint64_t)float_key(v[i]) << 32) | (uint32_t)~(uint32_t)e : 0ull;
  }
  // Sort the lane's keys, descending.
  topk_cas(key[0], key[1]); topk_cas(key[2], key[3]); topk_cas(key[4], key[5]); topk_cas(key[6], key[7]);
  topk_cas(key[0], key[2]); topk_cas(key[1], key[3]); topk_cas(key[4], key[6]); topk_cas(key[5], key[7]);
  topk_cas(key[1], key[2]); topk_cas(key[5], key[6]);
  topk_cas(key[0], key[4]); topk_cas(key[1], key[5]); topk_cas(key[2], key[6]); topk_cas(key[3], key[7]);
  topk_cas(key[2], key[4]); topk_cas(key[3], key[5]);
  topk_cas(key[1], key[2]); topk_cas(key[3], key[4]); topk_cas(key[5], key[6]);
  topk_merge_round<0xB1>(key);   // quad_perm [1,0,3,2]
  topk_merge_round<0x4E>(key);   // quad_perm [2,3,0,1]
  topk_merge_round<0x124>(key);  // row_ror:4
  topk_merge_round<0x128>(key);  // row_ror:8
  // Softmax over the row's experts, then the k selected probabilities.
  const float mx = key_float((uint32_t)(key[0] >> 32));
  float sl = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sl += v[i] == -INFINITY ? 0.f : __expf(v[i] - mx);
  const float s = row_fsum16(sl);
  float my_p = 0.f, psum = 0.f;
  int my_id = 0;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if (r < k) {
      const float p = __expf(key_float((uint32_t)(key[r] >> 32)) - mx) / s;
      psum += p;
      if (j == r) {
        my_p = p;
        my_id = (int)~(uint32_t)key[r];
      }
    }
  }
  if (tok >= 0 && j < k) emit(tok, j, my_id, renorm ? my_p / psum : my_p);
}

}  // namespace mstar
