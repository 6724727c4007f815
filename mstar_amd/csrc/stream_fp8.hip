// Persistent weight-streaming grouped GEMM for decode-sized FP8 MoE layers.
//
// At decode (a few tokens per expert) the layer is a pure weight stream:
// ~115 of 128 experts are hit and each expert's 4.7 MB of FP8 weights is
// read once.  This kernel is built for that regime:
//
//  * persistent: the grid is four 4-wave workgroups per CU; the work list is
//    the set of "wave items" (active expert, 16 weight rows) enumerated
//    expert-major, and every workgroup takes one contiguous range of it, so
//    a workgroup touches one or two experts and streams contiguous weight
//    rows;
//  * the active-expert list is built in each workgroup from the per-expert
//    counts the align kernel wrote (no host round trip, graph-capturable);
//  * a wave issues the weight fragments of up to eight 128-wide K steps of
//    an item at once (16 KB per wave) and runs their MFMAs as they land;
//    sixteen resident waves per CU keep ~256 KB of loads outstanding, which
//    is what hides HBM latency (straight-line code, no intra-wave
//    double-buffering, so the VGPR budget allows that occupancy);
//  * the token rows of the covered expert (16 per pass) are gathered, quantised per
//    128-group to e4m3fn (the same arithmetic as the standalone quant
//    kernel) and kept in LDS with their scales; weight-block scales are
//    loaded with the weight fragments;
//  * each v_mfma_f32_16x16x128_f8f6f4 covers exactly one 128-wide scale
//    block, so its fp32 partial is scaled by s_a[row] * s_w[block] and added.
// Epilogues: fused SiLU/GeLU-and-mul into the [slots, I] intermediate (gate
// and up rows of one output column sit in lanes l and l+8), or the down
// projection times the routed weight into [slots, H] (the reference's
// fused_moe_kernel with MUL_ROUTED_WEIGHT, kernels.py:129-138).
#include "common.h"
#include "launch.h"

namespace mstar {

constexpr int kStreamRows = 16;   // token rows staged per pass (one MFMA row block)
constexpr int kStreamWaves = 4;   // waves per workgroup
constexpr int kStreamWgPerCu = 4; // resident workgroups per CU (LDS ~35 KB each)
constexpr int kStreamSlotsPerThread = 4;  // ids mode: up to 1024 slots per launch

__device__ inline v8i lds_v8i(const uint8_t* p) {
  v4i lo = *(const v4i*)p, hi = *(const v4i*)(p + 16);
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Eight e4m3fn bytes (two dwords) -> one bf16x8 MFMA operand, exactly
// (e4m3fn is a subset of bf16).  Whole 32-bit pairs are moved: pulling
// single __bf16 elements out of the packed result makes the compiler insert
// byte permutes that scramble the pairs.
__device__ inline v8s fp8x8_to_bf16x8(int x0, int x1) {
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  const int c0 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)x0, 1.0f, false));
  const int c1 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)x0, 1.0f, true));
  const int c2 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)x1, 1.0f, false));
  const int c3 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)x1, 1.0f, true));
  return __builtin_bit_cast(v8s, v4i{c0, c1, c2, c3});
}

// One 16x16x128 block product of e4m3fn fragments.  EXACT: the fragments
// are widened to bf16 (exactly) and reduced by four chained bf16 MFMAs,
// whose fp32 accumulation is exact to fp32 rounding; otherwise one
// v_mfma_f32_16x16x128_f8f6f4, whose internal reduction of the 128
// products keeps fewer bits (partial sums can be off by ~1e-5 relative).
template <bool EXACT>
__device__ inline v4f block_dot_fp8(const v8i& a, const v8i& b) {
  if constexpr (!EXACT) {
    return mfma_fp8_16x16x128(a, b, v4f{0.f, 0.f, 0.f, 0.f});
  } else {
    v4f t = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      t = mfma_bf16_16x16x32(fp8x8_to_bf16x8(a[2 * s], a[2 * s + 1]),
                             fp8x8_to_bf16x8(b[2 * s], b[2 * s + 1]), t);
    return t;
  }
}

template <int EPI, int KS, bool EXACT>
__global__ __launch_bounds__(256) void stream_fp8_kernel(GemmArgs p) {
  constexpr int K = KS * 128;
  constexpr int KC = KS <= 6 ? KS : (KS % 4 == 0 ? 4 : (KS % 3 == 0 ? 3 : KS));  // K steps loaded at once
  constexpr int CH = KS / KC;                                   // loads per item
  constexpr int LDA = K + 16;
  constexpr int RC = kStreamRows;
  static_assert(KS % KC == 0, "KS must split into equal chunks");

  extern __shared__ __align__(16) uint8_t smem[];
  const int E = p.num_experts;
  uint8_t* sA = smem;                      // [RC][LDA] e4m3fn rows
  float* sAs = (float*)(sA + RC * LDA);    // [KS][RC] row scales (transposed)
  int* sSlot = (int*)(sAs + KS * RC);      // [RC] slot id of each staged row
  int* sAct = sSlot + RC;                  // [E] active experts, ascending
  int* sCnt = sAct + E;                    // [E] slots per expert
  int* sOff = sCnt + E;                    // [E] first slot-list entry per expert
  int* sList = sOff + E;                   // [numel] slots grouped by expert (ids mode)
  __shared__ int sNact;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const bool ids_mode = p.topk_ids != nullptr;

  // ---- per-expert slot lists.  ids mode: built here from topk_ids (the
  // order of slots inside an expert is irrelevant: every slot's outputs are
  // computed independently).  Otherwise: the align kernel's offsets, counts
  // and sorted_ids.
  if (ids_mode) {
    for (int e = tid; e < E; e += 256) sCnt[e] = 0;
    __syncthreads();
    int my_e[kStreamSlotsPerThread], my_pos[kStreamSlotsPerThread];
#pragma unroll
    for (int j = 0; j < kStreamSlotsPerThread; ++j) {
      const int i = tid + j * 256;
      int e = -1;
      if (i < p.M) {
        const int64_t v = p.ids_dtype == kI64 ? ((const int64_t*)p.topk_ids)[i]
                                              : (int64_t)((const int32_t*)p.topk_ids)[i];
        e = (v >= 0 && v < E) ? (int)v : -1;  // out-of-range ids are skipped (.cu:44-46)
      }
      my_e[j] = e;
      my_pos[j] = e >= 0 ? atomicAdd(&sCnt[e], 1) : 0;
    }
    __syncthreads();
    if (w == 0) {
      int run = 0;
      for (int e0 = 0; e0 < E; e0 += 64) {
        const int e = e0 + lane;
        const int c = e < E ? sCnt[e] : 0;
        const int incl = wave_incl_scan(c);
        if (e < E) sOff[e] = run + incl - c;
        run += __shfl(incl, 63, 64);
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kStreamSlotsPerThread; ++j)
      if (my_e[j] >= 0) sList[sOff[my_e[j]] + my_pos[j]] = tid + j * 256;
  } else {
    for (int e = tid; e < E; e += 256) {
      sCnt[e] = p.expert_cnt[e];
      sOff[e] = p.expert_off[e];
    }
  }
  __syncthreads();
  // ---- active experts, ascending
  if (w == 0) {
    int n = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const bool act = e < E && sCnt[e] > 0;
      const uint64_t b = __ballot(act);
      if (act) sAct[n + __builtin_popcountll(b & ((1ull << lane) - 1ull))] = e;
      n += __builtin_popcountll(b);
    }
    if (lane == 0) sNact = n;
  }
  __syncthreads();
  const int n_act = sNact;
  const int IPE = EPI == EPI_ACT ? p.inter / 8 : p.N / 16;  // wave items per expert
  const int total = n_act * IPE;
  const int T = (total + gridDim.x - 1) / gridDim.x;
  const int i0 = blockIdx.x * T;
  const int i1 = i0 + T < total ? i0 + T : total;
  if (i0 >= i1) return;

  const uint16_t* A16 = (const uint16_t*)p.A;
  uint16_t* C = (uint16_t*)p.C;

  for (int a = i0 / IPE; a * IPE < i1; ++a) {
    const int e = sAct[a];
    const int cnt = sCnt[e];
    const int off = sOff[e];
    const int ia0 = i0 > a * IPE ? i0 : a * IPE;
    const int ia1 = i1 < (a + 1) * IPE ? i1 : (a + 1) * IPE;
    const uint8_t* Be = (const uint8_t*)p.B + (int64_t)e * p.b_estride;
    const float* Se = (const float*)p.b_scale + (int64_t)e * p.bs_estride;

    for (int r0 = 0; r0 < cnt; r0 += RC) {
      const int rows = cnt - r0 < RC ? cnt - r0 : RC;
      __syncthreads();  // the previous pass is done with LDS
      // ---- gather + quantise the expert's token rows into LDS
      const int groups = rows * KS;
      for (int g0 = 0; g0 < groups; g0 += 16) {
        const int gq = g0 + (tid >> 4), sub = tid & 15;
        const bool live = gq < groups;
        const int rr = live ? gq / KS : 0, kk = live ? gq % KS : 0;
        int slot = 0;
        if (live) slot = ids_mode ? sList[off + r0 + rr] : p.sorted_ids[off + r0 + rr];
        const int arow = slot / p.top_k;
        v4i raw = live ? *(const v4i*)(A16 + (int64_t)arow * p.lda + kk * 128 + sub * 8)
                       : v4i{0, 0, 0, 0};
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f[2 * i] = bf16_bits_to_f32((uint16_t)(raw[i] & 0xffff));
          f[2 * i + 1] = bf16_bits_to_f32((uint16_t)((uint32_t)raw[i] >> 16));
        }
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
        amax = group_max<16>(amax);
        const float sc = fmaxf(amax, kQuantEps) / kFp8Max;
        const int lo = cvt_fp8x4(clamp_fp8(f[0] / sc), clamp_fp8(f[1] / sc),
                                 clamp_fp8(f[2] / sc), clamp_fp8(f[3] / sc));
        const int hi = cvt_fp8x4(clamp_fp8(f[4] / sc), clamp_fp8(f[5] / sc),
                                 clamp_fp8(f[6] / sc), clamp_fp8(f[7] / sc));
        if (live) {
          *(int2*)(sA + rr * LDA + kk * 128 + sub * 8) = make_int2(lo, hi);
          if (sub == 0) {
            sAs[kk * RC + rr] = sc;
            if (kk == 0) sSlot[rr] = slot;
          }
        }
      }
      // rows beyond `rows`: zero scales (their A fragments are zeroed on read)
      for (int i = tid; i < KS * RC; i += 256)
        if (i % RC >= rows) sAs[i] = 0.f;
      __syncthreads();

      const bool arow_ok = l16 < rows;
      for (int it = ia0 + w; it < ia1; it += kStreamWaves) {
        const int g = it - a * IPE;
        int br;
        if constexpr (EPI == EPI_ACT) {
          const int ocol = g * 8 + (l16 & 7);
          br = l16 < 8 ? ocol : p.inter + ocol;
        } else {
          br = g * 16 + l16;
        }
        const uint8_t* src = Be + (int64_t)br * p.ldb + lg * 32;
        const float* ss = Se + (int64_t)(br / 128) * p.bs_ld;
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
        for (int c = 0; c < CH; ++c) {
          v8i b[KC];
          float sw[KC];
#pragma unroll
          for (int kk = 0; kk < KC; ++kk) {
            b[kk] = *(const v8i*)(src + (c * KC + kk) * 128);
            sw[kk] = ss[c * KC + kk];
          }
#pragma unroll
          for (int kk = 0; kk < KC; ++kk) {
            const int kg = c * KC + kk;
            v8i af = arow_ok ? lds_v8i(sA + l16 * LDA + kg * 128 + lg * 32)
                             : v8i{0, 0, 0, 0, 0, 0, 0, 0};
            v4f t = block_dot_fp8<EXACT>(af, b[kk]);
            v4f sa = *(const v4f*)(sAs + kg * RC + lg * 4);
            acc += t * (sa * sw[kk]);
          }
        }
        // ---- epilogue of item g
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int orow = lg * 4 + r;
          const float mine = acc[r];
          if constexpr (EPI == EPI_ACT) {
            const float up = __shfl_xor(mine, 8, 64);
            if (orow < rows && l16 < 8) {
              const int slot = sSlot[orow];
              const float gg = round_bf16(mine);
              const float u = round_bf16(up);
              const float av = round_bf16(p.activation == 0 ? act_f32<0>(gg) : act_f32<1>(gg));
              C[(int64_t)slot * p.ldc + g * 8 + l16] = f32_to_bf16_bits(av * u);
            }
          } else {
            if (orow < rows) {
              const int slot = sSlot[orow];
              const float rw = p.mul_routed ? load_weight_any(p.topk_w, p.topk_w_dtype, slot) : 1.f;
              C[(int64_t)slot * p.ldc + g * 16 + l16] = f32_to_bf16_bits(mine * rw);
            }
          }
        }
      }
    }
  }
}

static int g_num_cu = 0;

static int num_cu() {
  if (g_num_cu <= 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_num_cu = n;
  }
  return g_num_cu;
}

template <int EPI, int KS, bool EXACT>
static int run_stream_fp8(const GemmArgs& a, hipStream_t stream) {
  constexpr int K = KS * 128;
  const size_t shmem = (size_t)kStreamRows * (K + 16) + (size_t)KS * kStreamRows * 4 +
                       kStreamRows * 4 + (size_t)a.num_experts * 3 * 4 +
                       (a.topk_ids ? (size_t)a.M * 4 : 0);
  auto kern = stream_fp8_kernel<EPI, KS, EXACT>;
  static size_t attr_bytes = 0;  // largest LDS size opted in so far
  if (shmem > attr_bytes) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)shmem) != hipSuccess) {
      set_last_error("stream_fp8: cannot reserve %zu bytes of LDS", shmem);
      return kLaunchError;
    }
    attr_bytes = shmem;
  }
  const int grid = kStreamWgPerCu * num_cu();
  kern<<<dim3(grid), dim3(256), shmem, stream>>>(a);
  return launch_status("stream_fp8");
}

bool stream_fp8_supported(int K, int N, int inter, int epi) {
  if (K % 128 != 0) return false;
  const int ks = K / 128;
  const bool ks_ok = ks == 1 || ks == 2 || ks == 3 || ks == 4 || ks == 6 || ks == 8 || ks == 12 || ks == 16;
  const bool n_ok = epi == EPI_ACT ? inter % 8 == 0 : N % 16 == 0;
  return ks_ok && n_ok;
}

int launch_stream_fp8(const GemmArgs& a, int epi, bool exact, hipStream_t stream) {
  if (!stream_fp8_supported(a.K, a.N, a.inter, epi) || a.num_experts > 1024 ||
      (a.topk_ids && a.M > kStreamMaxIdsSlots)) {
    set_last_error("stream_fp8: unsupported shape (K=%d N=%d slots=%lld)", a.K, a.N, (long long)a.M);
    return kUnsupported;
  }
#define MSTAR_SF8(KS)                                                                       \
  case KS:                                                                                  \
    if (exact)                                                                              \
      return epi == EPI_ACT ? run_stream_fp8<EPI_ACT, KS, true>(a, stream)                  \
                            : run_stream_fp8<EPI_STORE, KS, true>(a, stream);               \
    return epi == EPI_ACT ? run_stream_fp8<EPI_ACT, KS, false>(a, stream)                   \
                          : run_stream_fp8<EPI_STORE, KS, false>(a, stream);
  switch (a.K / 128) {
    MSTAR_SF8(1)
    MSTAR_SF8(2)
    MSTAR_SF8(3)
    MSTAR_SF8(4)
    MSTAR_SF8(6)
    MSTAR_SF8(8)
    MSTAR_SF8(12)
    MSTAR_SF8(16)
  }
#undef MSTAR_SF8
  return kUnsupported;
}

}  // namespace mstar
