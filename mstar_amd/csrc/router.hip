// Fused router: logits = x . Wg^T (bf16 operands, fp32 accumulation, bf16
// result), fp32 softmax, top-k, optional renormalisation -- one launch.
// Restates TopKRouter.forward (mstar/model/components/moe.py:130-140):
// F.linear in bf16, F.softmax(dtype=float), torch.topk, w / sum(w).
//
// A workgroup of 8 waves owns 16 tokens.  Wave w computes expert tiles
// w, w + 8, ... of 16 experts with v_mfma_f32_16x16x32_bf16 (experts as the
// MFMA's A operand, tokens as B), streaming its Wg rows and the 16 token
// rows straight from global memory in 16-byte pieces, four K-steps in
// flight.  The bf16-rounded logits go to LDS (and, if asked, to logits_out);
// then each wave ranks two tokens with the same wave top-k as the routing
// kernels.
#include "common.h"
#include "launch.h"
#include "topk.h"

namespace mstar {

constexpr int kRouterTokens = 16;
constexpr int kRouterWaves = 8;
constexpr int kRouterMaxE = 256;

template <int EPL>
__global__ __launch_bounds__(kRouterWaves * 64) void router_kernel(
    const uint16_t* __restrict__ x, int64_t M, int H, const uint16_t* __restrict__ wg, int E, int k,
    int renorm, float* __restrict__ w_out, int32_t* __restrict__ ids32, int64_t* __restrict__ ids64,
    uint16_t* __restrict__ logits_out) {
  __shared__ float sL[kRouterTokens][kRouterMaxE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * kRouterTokens;
  const int64_t tok = t0 + l16;
  const bool tok_ok = tok < M;
  const uint16_t* xrow = x + (tok_ok ? tok : 0) * (int64_t)H + lg * 8;
  const int ntiles = (E + 15) / 16;
  for (int tile = wave; tile < ntiles; tile += kRouterWaves) {
    const int e = tile * 16 + l16;
    const bool e_ok = e < E;
    const uint16_t* wrow = wg + (int64_t)(e_ok ? e : 0) * H + lg * 8;
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    constexpr int kIn = 4;  // K-steps of 32 loaded ahead
    for (int k0 = 0; k0 < H; k0 += 32 * kIn) {
      v8s a[kIn], b[kIn];
#pragma unroll
      for (int s = 0; s < kIn; ++s) {
        const int kk = k0 + 32 * s;
        const bool in = kk < H;
        a[s] = in && e_ok ? *(const v8s*)(wrow + kk) : v8s{};
        b[s] = in && tok_ok ? *(const v8s*)(xrow + kk) : v8s{};
      }
#pragma unroll
      for (int s = 0; s < kIn; ++s) acc = mfma_bf16_16x16x32(a[s], b[s], acc);
    }
    // Lane (l16, lg) holds experts tile*16 + 4 lg + r of token t0 + l16.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int er = tile * 16 + 4 * lg + r;
      const uint16_t bits = f32_to_bf16_bits(acc[r]);
      if (er < E) {
        sL[l16][er] = bf16_bits_to_f32(bits);
        if (logits_out && tok_ok) logits_out[tok * E + er] = bits;
      }
    }
  }
  __syncthreads();
  for (int tl = wave; tl < kRouterTokens; tl += kRouterWaves) {
    const int64_t t = t0 + tl;
    if (t >= M) break;
    float v[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = j * 64 + lane;
      v[j] = e < E ? sL[tl][e] : -INFINITY;
    }
    topk_wave<EPL>(v, E, k, renorm, lane, [&](int r, int id, float wt) {
      w_out[t * k + r] = wt;
      if (ids32) ids32[t * k + r] = id;
      if (ids64) ids64[t * k + r] = id;
    });
  }
}

int launch_router(const void* hidden, int64_t M, int64_t H, const void* gate_weight, int E, int k,
                  int renorm, float* w, int32_t* ids32, int64_t* ids64, void* logits_out,
                  hipStream_t stream) {
  if (M < 0 || H <= 0 || H % 32 != 0 || H > INT32_MAX || E <= 0 || E > kRouterMaxE || k <= 0 ||
      k > E || k > 64 || (M > 0 && (!w || (!ids32 && !ids64) || !hidden || !gate_weight))) {
    set_last_error("router: invalid arguments (M=%lld H=%lld E=%d k=%d; H %% 32 == 0, E <= %d)",
                   (long long)M, (long long)H, E, k, kRouterMaxE);
    return kInvalidArgument;
  }
  if (M == 0) return kOk;
  const dim3 grid((unsigned)((M + kRouterTokens - 1) / kRouterTokens)), block(kRouterWaves * 64);
  const uint16_t* x = (const uint16_t*)hidden;
  const uint16_t* wg = (const uint16_t*)gate_weight;
  uint16_t* lo = (uint16_t*)logits_out;
  const int epl = (E + 63) / 64;
  if (epl <= 1)
    router_kernel<1><<<grid, block, 0, stream>>>(x, M, (int)H, wg, E, k, renorm, w, ids32, ids64, lo);
  else if (epl <= 2)
    router_kernel<2><<<grid, block, 0, stream>>>(x, M, (int)H, wg, E, k, renorm, w, ids32, ids64, lo);
  else
    router_kernel<4><<<grid, block, 0, stream>>>(x, M, (int)H, wg, E, k, renorm, w, ids32, ids64, lo);
  return launch_status("router");
}

}  // namespace mstar
