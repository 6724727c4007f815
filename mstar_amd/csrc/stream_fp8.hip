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
#include <atomic>

#include "common.h"
#include "launch.h"
#include "layer_sync.h"

namespace mstar {

constexpr int kStreamRows = 16;   // token rows staged per pass (one MFMA row block)
constexpr int kStreamWaves = 4;   // waves per workgroup
constexpr int kStreamWgPerCu = 4; // resident workgroups per CU (LDS ~35 KB each)
constexpr int kGatherBatchQ = 4;          // 16-byte row pieces in flight per thread (FP8 rows)
constexpr int kGatherBatchH = 3;          // groups in flight per 16 lanes (bf16 rows)

__device__ inline v8i lds_v8i(const uint8_t* p) {
  v4i lo = *(const v4i*)p, hi = *(const v4i*)(p + 16);
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ inline v8s fp8x8_to_bf16x8(int x0, int x1) {
  return __builtin_bit_cast(v8s, fp8x8_to_bf16x8_bits(x0, x1));
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

// Per-expert slot lists in LDS.  ids mode (p.topk_ids set): built from the
// router ids (the order of slots inside an expert is irrelevant: every
// slot's outputs are computed independently).  Otherwise: the align
// kernel's offsets, counts and sorted_ids.  Then the active experts,
// ascending, and their number.  Ends with a barrier.
template <int NT>
__device__ __forceinline__ void build_expert_lists(const GemmArgs& p, int tid, int w, int lane,
                                                   int* sAct, int* sCnt, int* sOff, int* sList,
                                                   int* nact) {
  constexpr int SPT = (int)(kStreamMaxIdsSlots / NT);  // slots per thread
  const int E = p.num_experts;
  // ---- per-expert slot lists.  ids mode: built here from topk_ids (the
  // order of slots inside an expert is irrelevant: every slot's outputs are
  // computed independently).  Otherwise: the align kernel's offsets, counts
  // and sorted_ids.
  if (p.topk_ids) {
    for (int e = tid; e < E; e += NT) sCnt[e] = 0;
    __syncthreads();
    int my_e[SPT], my_pos[SPT];
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const int i = tid + j * NT;
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
        run += wave_last(incl);
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SPT; ++j)
      if (my_e[j] >= 0) sList[sOff[my_e[j]] + my_pos[j]] = tid + j * NT;
  } else {
    for (int e = tid; e < E; e += NT) {
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
    if (lane == 0) *nact = n;
  }
  __syncthreads();
}

template <int EPI, int KS, bool EXACT, bool AQ>
__global__ __launch_bounds__(256) void stream_fp8_kernel(GemmArgs p) {
  constexpr int K = KS * 128;
  // K-steps per chunk; two chunks are in flight per wave.
  constexpr int KC = KS % 2 == 0 ? 2 : (KS % 3 == 0 ? 3 : 1);
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

  build_expert_lists<256>(p, tid, w, lane, sAct, sCnt, sOff, sList, &sNact);
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
    // This wave's work in the expert: items ia0 + w, ia0 + w + 4, ...; each
    // item is CH chunks of KC K-steps.  q enumerates (item, chunk) pairs.
    const int my_items = ia0 + w < ia1 ? (ia1 - ia0 - w + kStreamWaves - 1) / kStreamWaves : 0;
    const int nq = my_items * CH;

    // Weight row of this lane for item `it`.
    auto weight_row = [&](int it) -> int {
      const int g = it - a * IPE;
      if constexpr (EPI == EPI_ACT) {
        const int ocol = g * 8 + (l16 & 7);
        return l16 < 8 ? ocol : p.inter + ocol;
      } else {
        return g * 16 + l16;
      }
    };
    // Loads of chunk q: KC weight fragments (32 bytes per lane and K-step)
    // and their block scales.
    auto load_chunk = [&](int q, v8i (&bq)[KC], float (&sq)[KC]) {
      const int it = ia0 + w + (q / CH) * kStreamWaves, c = q % CH;
      const int br = weight_row(it);
      const uint8_t* src = Be + (int64_t)br * p.ldb + lg * 32 + c * KC * 128;
      const float* ss = Se + (int64_t)(br / 128) * p.bs_ld + c * KC;
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        bq[kk] = *(const v8i*)(src + kk * 128);
        sq[kk] = ss[kk];
      }
    };

    for (int r0 = 0; r0 < cnt; r0 += RC) {
      const int rows = cnt - r0 < RC ? cnt - r0 : RC;
      // Two register buffers: chunk q+1 is in flight while chunk q computes.
      // The first chunk is issued before the token gather so its latency
      // overlaps the gather and the barrier.
      v8i b0[KC], b1[KC];
      float s0[KC], s1[KC];
      if (nq > 0) load_chunk(0, b0, s0);
      __syncthreads();  // the previous pass is done with LDS
      // ---- stage the expert's token rows (e4m3fn) and group scales in LDS.
      // All loads of a batch are issued before any is used.
      auto slot_of = [&](int rr) { return ids_mode ? sList[off + r0 + rr] : p.sorted_ids[off + r0 + rr]; };
      if constexpr (AQ) {
        // Pre-quantised rows: a copy.
        constexpr int PPR = K / 16;  // 16-byte pieces per row
        constexpr int B = kGatherBatchQ;
        const int pieces = rows * PPR;
        const uint8_t* A8 = (const uint8_t*)p.A;
        for (int base = 0; base < pieces; base += 256 * B) {
          v4i v[B];
#pragma unroll
          for (int j = 0; j < B; ++j) {
            const int pc = base + j * 256 + tid;
            const int rr = pc / PPR, c = pc % PPR;
            v[j] = pc < pieces ? *(const v4i*)(A8 + (int64_t)(slot_of(rr) / p.top_k) * p.lda + c * 16)
                               : v4i{0, 0, 0, 0};
          }
#pragma unroll
          for (int j = 0; j < B; ++j) {
            const int pc = base + j * 256 + tid;
            const int rr = pc / PPR, c = pc % PPR;
            if (pc < pieces) *(v4i*)(sA + rr * LDA + c * 16) = v[j];
          }
        }
        for (int i = tid; i < rows * KS; i += 256) {
          const int rr = i / KS, kk = i % KS;
          const int slot = slot_of(rr);
          sAs[kk * RC + rr] = p.a_scale[(int64_t)(slot / p.top_k) * p.ld_as + kk];
          if (kk == 0) sSlot[rr] = slot;
        }
      } else {
        // bf16 rows, quantised per group of 128 here (16 lanes per group).
        constexpr int B = kGatherBatchH;
        const int groups = rows * KS;
        for (int g0 = 0; g0 < groups; g0 += 16 * B) {
          v4i raw[B];
          int slots[B];
#pragma unroll
          for (int j = 0; j < B; ++j) {
            const int gq = g0 + j * 16 + (tid >> 4), sub = tid & 15;
            const bool live = gq < groups;
            const int rr = live ? gq / KS : 0, kk = live ? gq % KS : 0;
            slots[j] = live ? slot_of(rr) : 0;
            raw[j] = live ? *(const v4i*)(A16 + (int64_t)(slots[j] / p.top_k) * p.lda + kk * 128 + sub * 8)
                          : v4i{0, 0, 0, 0};
          }
#pragma unroll
          for (int j = 0; j < B; ++j) {
            const int gq = g0 + j * 16 + (tid >> 4), sub = tid & 15;
            const bool live = gq < groups;
            const int rr = live ? gq / KS : 0, kk = live ? gq % KS : 0;
            float sc;
            const int2 codes = quant_group8<kBF16>(raw[j], sc);
            if (live) {
              *(int2*)(sA + rr * LDA + kk * 128 + sub * 8) = codes;
              if (sub == 0) {
                sAs[kk * RC + rr] = sc;
                if (kk == 0) sSlot[rr] = slots[j];
              }
            }
          }
        }
      }
      // rows beyond `rows`: zero scales (their A fragments are zeroed on read)
      for (int i = tid; i < KS * RC; i += 256)
        if (i % RC >= rows) sAs[i] = 0.f;
      __syncthreads();

      const bool arow_ok = l16 < rows;
      v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
      // Chunk q: MFMAs of its KC K-steps; after an item's last chunk, the
      // item's epilogue.
      auto compute = [&](int q, const v8i (&bq)[KC], const float (&sq)[KC]) {
        const int it = ia0 + w + (q / CH) * kStreamWaves, c = q % CH;
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) {
          const int kg = c * KC + kk;
          v8i af = arow_ok ? lds_v8i(sA + l16 * LDA + kg * 128 + lg * 32)
                           : v8i{0, 0, 0, 0, 0, 0, 0, 0};
          v4f t = block_dot_fp8<EXACT>(af, bq[kk]);
          v4f sa = *(const v4f*)(sAs + kg * RC + lg * 4);
          acc += t * (sa * sq[kk]);
        }
        if (c != CH - 1) return;
        const int g = it - a * IPE;
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
        acc = v4f{0.f, 0.f, 0.f, 0.f};
      };
#pragma unroll 1
      for (int q = 0; q < nq; q += 2) {
        if (q + 1 < nq) load_chunk(q + 1, b1, s1);
        compute(q, b0, s0);
        if (q + 1 >= nq) break;
        if (q + 2 < nq) load_chunk(q + 2, b0, s0);
        compute(q + 1, b1, s1);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// CU-resident variant (exact FP8, router-ids mode): one 512-thread
// workgroup per CU, and every CU takes an equal contiguous range of items
// (16 weight rows of one hit expert each).  Such a range spans at most two
// experts at decode shapes.
//  * Activation rows: the CU stages the rows of its experts' slots (A row =
//    slot / top_k) in LDS once, quantised per group of 128 and widened to
//    bf16 (e4m3fn is a subset of bf16): copied from pre-quantised widened
//    rows (STAGE_Q16, as the routing launch writes them) or quantised here
//    from bf16 (STAGE_H16).  Row sets beyond the LDS budget are processed in
//    windows.
//  * Weights: each wave streams its items through a private three-slot LDS
//    ring with LDS-DMA loads (global_load_lds_dwordx4).  One instruction
//    fetches 8 weight rows x 128 bytes -- whole 128-byte lines, the access
//    shape that streams fastest -- with the streaming cache policy; the 16
//    bytes of lane l land at slot + 16 l (row l / 8, physical chunk l % 8,
//    holding logical chunk (l % 8) ^ row, so the fragment reads below are
//    bank-conflict free).  Two chunks are in flight while one computes; the
//    waits are per wave (vmcnt), so the main loop has no workgroup barrier.
//  * Math: lane l reads weight row l % 16, K bytes 32 (l / 16) .. +31 of a
//    K-step from the ring (MFMA A operand) and the matching 32 bf16 token
//    values from the staged rows (B operand: token row l % 16 of the
//    expert).  Weights are widened exactly to bf16; each 128-wide block is
//    four bf16 MFMAs with exact fp32 accumulation, scaled by
//    s_token[block] * s_weight[block].  Lane l ends with (weight rows
//    4 (l/16) .. +3) x (token l % 16).  Lanes past the expert's token count
//    read row 0 and store nothing (MFMA output columns are independent).
// STAGE_W4: W4A16 -- int4 weights (group-128 bf16 scales whose products
// with the codes are exact in bf16) and bf16 token rows, staged with each
// group of 8 reordered to the codes' unpacked order (int4x8_bias128) and
// with each 128-element block's sum.
enum : int { STAGE_Q16 = 0, STAGE_H16 = 1, STAGE_W4 = 2 };
constexpr int kCuThreads = 512;
// int4 weights: sixteen waves per CU (their rings are half the size), so
// that more waves' dependent LDS / VALU / MFMA chains overlap.
constexpr int kCuThreadsW4 = 1024;
template <bool W4>
__host__ __device__ constexpr int cu_waves() { return (W4 ? kCuThreadsW4 : kCuThreads) / 64; }
constexpr int kCuRing = 3;        // ring slots per wave
constexpr size_t kCuLdsMax = 160 * 1024;
constexpr int kDmaAux = 2;        // cache policy of the weight stream (streaming)

template <int KS>
__host__ __device__ constexpr int cu_kc() { return KS % 2 == 0 ? 2 : KS; }  // K-steps per chunk
template <int KS>
__host__ __device__ constexpr int cu_pitch() { return KS * 256 + 16; }     // bytes per staged bf16 row
// int4 weights: K-steps per chunk (a 128-byte line of a row holds two), and
// the ring slot: KC / 2 lines of 16 rows, then the rows' KC bf16 scales.
template <int KS>
__host__ __device__ constexpr int cu_w4_kc() { return 2; }
template <int KS>
__host__ __device__ constexpr int cu_w4_slot() { return cu_w4_kc<KS>() * (1024 + 32); }
template <int KS, bool W4 = false>
__host__ __device__ constexpr size_t cu_ring_bytes() {
  return (size_t)cu_waves<W4>() * kCuRing * (W4 ? cu_w4_slot<KS>() : cu_kc<KS>() * 2048);
}
// LDS layout: rings | sAct[E] sCnt[E] sOff[E] sList[M'] sMask[32] sFlags[kFlagWords]
// | sSc[cap][KS] sRw[cap] | rows[cap][pitch].  The lists sit at the same offset for every KS
// with the same ring size, so the layout kernel's down phase reuses the
// gate_up phase's lists.
// sFlags (the layer kernel's per-workgroup words): [0] the workgroup's own
// gate_up range is its to run, [1] the current down window's wait gave up,
// [2] ranges stolen, [3 ..) their indices.
constexpr int kFlagOwn = 0, kFlagPoison = 1, kFlagStealN = 2, kFlagSteal = 3;
constexpr int kMaxSteals = 256;
constexpr int kFlagWords = kFlagSteal + kMaxSteals + 1;
__host__ __device__ inline size_t cu_lists_bytes(int E, int64_t M) {
  return ((size_t)3 * E + (size_t)((M + 3) & ~3ll) + 32 + kFlagWords) * 4;
}
template <int KS, bool W4 = false>
__host__ __device__ inline size_t cu_sc_off(int E, int64_t M, size_t lists_at = 0) {
  return (lists_at ? lists_at : cu_ring_bytes<KS, W4>()) + cu_lists_bytes(E, M);
}
template <int KS, bool W4 = false>
__host__ __device__ inline size_t cu_rows_off(int E, int64_t M, int cap, size_t lists_at = 0) {
  return (cu_sc_off<KS, W4>(E, M, lists_at) + (size_t)cap * (KS + 1) * 4 + 15) & ~(size_t)15;
}

// Wait for the oldest of `ahead` chunks in flight (DPC DMA instructions
// each), leaving the younger ones -- two instructions fewer, for the
// epilogue store or routed-weight load that may sit between them:
// over-waiting is safe.
template <int DPC, int N>
__device__ __forceinline__ void wait_leaving_chunks(int ahead) {
  if constexpr (N >= 2) {
    if (ahead >= N) {
      wait_vmcnt<((N - 1) * DPC - 2 > 0 ? (N - 1) * DPC - 2 : 0)>();
      return;
    }
    wait_leaving_chunks<DPC, N - 1>(ahead);
  } else {
    wait_vmcnt<0>();
  }
}

// Swizzle of the 16-byte pieces of int4 ring row r (rows 128 bytes apart):
// the 16 rows' reads of one logical piece fall in distinct banks.
__device__ __forceinline__ int w4_swz(int r) { return (r >> 1) & 7; }

// 16 bytes of 16-bit row data; COHERENT: as two agent-scope atomic loads,
// which see other XCDs' agent-scope atomic stores without an L2 invalidate.
template <bool COHERENT>
__device__ __forceinline__ v4i load_rows16(const uint16_t* p) {
  if constexpr (COHERENT) {
    const uint64_t lo = __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t hi = __hip_atomic_load((const uint64_t*)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return v4i{(int)(uint32_t)lo, (int)(uint32_t)(lo >> 32), (int)(uint32_t)hi, (int)(uint32_t)(hi >> 32)};
  } else {
    return *(const v4i*)p;
  }
}

// Phase timestamps of the streaming kernels (a timeline build only:
// compiled with MSTAR_TIMELINE, read back with mstar_debug_timeline).
#ifdef MSTAR_TIMELINE
__device__ uint64_t g_timeline[2 * 1024 * 8];  // [EPI][workgroup][phase]
#define MSTAR_TL(i)                                                                          \
  do {                                                                                       \
    if (threadIdx.x == 0) g_timeline[((EPI & 1) * 1024 + blockIdx.x) * 8 + (i)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define MSTAR_TL(i) \
  do {              \
  } while (0)
#endif

// The decode layer in one launch (stream_layer_kernel): the gate_up
// phase of a workgroup reports, per expert, the (item, token row) pairs it
// finished; the down phase stages an expert's activation rows only once
// all of that expert's gate_up pairs are reported.
enum : int { kPhaseAlone = 0, kPhaseGate = 1, kPhaseDown = 2 };
//
// Forward progress.  Gate_up range q belongs to whichever workgroup first
// claims it: claim word q goes 0 -> 1 (its own workgroup, early in its
// gate_up phase) or 0 -> 2 (a thief).  Only the claimant reports a range's
// rows.  At the end of its own gate_up items every workgroup tries to claim
// each gate_up range its down range depends on and runs the ones it wins
// before its down phase.  So before any down-phase wait, every range the
// wait depends on is claimed by a workgroup that is running and whose
// gate_up work never waits: every wait ends, even when some of the launch's
// workgroups are not resident (another kernel or process holds CUs).  A late
// workgroup whose range was taken stops within the unit it is in (rows it
// wrote get the same values from the thief) and goes on to its down work.  A
// wait longer than kLayerWaitTicks is therefore a fault, not a schedule: it
// sets *err, counts itself and writes NaN rows for the window it gave up on,
// so the output is detectably invalid, never silently wrong.
enum : int { kLayerNormal = 0, kLayerTestNoOwnClaim = 1, kLayerTestGiveUp = 2 };
struct LayerSync {
  int* done;       // [E] gate_up (item, token row) pairs finished per expert; zero at launch
  int* err;        // set to 1 if a wait gave up (output of that launch invalid)
  int* claim;      // claim word of gate_up range q at claim[q * kClaimStride]; zero at launch
  int gate_ipe;    // gate_up items per expert (inter / 8)
  int down_ipe;    // down items per expert (hidden / 16)
  int lists_at;    // LDS offset of the expert lists (after both phases' rings)
  int mode;        // kLayerNormal, or a test mode set from the host:
                   // kLayerTestNoOwnClaim: odd workgroups do not claim their own range
                   // (as if not yet resident), kLayerTestGiveUp: every wait gives up at once
};
constexpr int kClaimStride = 16;  // one claim word per 64 bytes
constexpr int kMaxLayerRanges = kLayerSyncMaxCus;  // workgroups of a layer launch (one per CU)
// Sync words: done[E], err, then the claim words from a 16-word boundary.
__host__ __device__ inline int layer_claim_base(int E) { return (E + 16) / 16 * 16; }
int layer_sync_words(int E, int nwg) { return layer_claim_base(E) + kClaimStride * nwg; }
// Test mode of the launches enqueued from now on (mstar_moe_debug_layer_test_mode).
static std::atomic<int> g_layer_test_mode{kLayerNormal};
int set_layer_test_mode(int mode) {
  if (mode != kLayerNormal && mode != kLayerTestNoOwnClaim && mode != kLayerTestGiveUp) {
    set_last_error("moe_debug_layer_test_mode: unknown mode %d", mode);
    return kInvalidArgument;
  }
  g_layer_test_mode.store(mode, std::memory_order_relaxed);
  return kOk;
}
// Waits of the layer kernel that gave up (kLayerWaitTicks), on this device,
// since the library was loaded: read by mstar_moe_layer_wait_failures.
__device__ int g_layer_wait_failures;
// Longest wait of the down phase for an expert's gate_up rows before it
// gives up (s_memrealtime ticks of 10 ns): 100 ms.
constexpr uint64_t kLayerWaitTicks = 10000000;

// One workgroup's share of a streaming GEMM: work range `wg` of `nwg`.
// Layer gate_up phase: `own` -- range wg is this workgroup's own (claimed
// here; the end of the phase also claims the ranges its down range waits
// on), else a range it already claimed as a thief.
template <int EPI, int KS, int STAGE, int PHASE = kPhaseAlone>
__device__ __forceinline__ void stream_cu_body(const GemmArgs& p, int cap, int wg, int nwg, const LayerSync& ls,
                                               bool own = true) {
  static_assert(PHASE == kPhaseAlone || (PHASE == kPhaseGate) == (EPI == EPI_ACT),
                "layer phases: gate_up, then down");
  constexpr bool W4 = STAGE == STAGE_W4;
  static_assert(!W4 || KS % 2 == 0, "int4 chunks are two K-steps");
  constexpr int PITCH = cu_pitch<KS>();
  constexpr int KC = W4 ? cu_w4_kc<KS>() : cu_kc<KS>();  // K-steps per chunk
  constexpr int CH = KS / KC;               // chunks per item
  // Ring slot: FP8 -- 16 rows x KC x 128 bytes; int4 -- KC / 2 lines (two
  // K-steps each) of the 16 rows as blocks of 8 rows x 128 bytes (pieces
  // swizzled), then the 16 rows' KC bf16 scales (2 KC bytes a row).
  constexpr int SLOT = W4 ? cu_w4_slot<KS>() : KC * 2048;
  constexpr int WAVE_RING = W4 ? kCuRing * SLOT : kCuRing * cu_kc<KS>() * 2048;  // ring bytes per wave
  constexpr int RING = WAVE_RING / SLOT;    // slots per wave
  constexpr int DPC = W4 ? KC + 1 : 2 * KC;  // DMA instructions per chunk
  constexpr int W4_PR = KC / 2;             // int4: 4-byte scale pieces per row
  static_assert(RING >= 3 && RING <= 6, "ring depth");
  constexpr int NTH = W4 ? kCuThreadsW4 : kCuThreads;  // threads of the workgroup
  constexpr int NWV = NTH / 64;                          // its waves
  constexpr int SPT = (int)(kStreamMaxIdsSlots / NTH);  // router ids per thread
  // Waves that stage activation rows; the others prefetch weights meanwhile.
  constexpr int SW = STAGE == STAGE_Q16 ? 2 : 4;
  typedef __attribute__((address_space(3))) void* lds_void_ptr;
  extern __shared__ __align__(16) uint8_t smem[];
  const int E = p.num_experts;
  // The layer kernel puts the lists after the larger of its two phases' rings.
  const size_t lists_at = PHASE == kPhaseAlone ? 0 : (size_t)ls.lists_at;
  int* sAct = (int*)(smem + (lists_at ? lists_at : cu_ring_bytes<KS, W4>()));
  int* sCnt = sAct + E;
  int* sOff = sCnt + E;
  int* sList = sOff + E;
  float* sSc = (float*)(smem + cu_sc_off<KS, W4>(E, p.M, lists_at));
  float* sRw = sSc + cap * KS;  // routed weight of each staged row
  uint8_t* sRows = smem + cu_rows_off<KS, W4>(E, p.M, cap, lists_at);
  uint32_t* sMask = (uint32_t*)(sList + ((p.M + 3) & ~3ll));  // [32] active experts (E <= 1024)
  int* sFlags = (int*)(sMask + 32);
  // The down phase of the layer kernel finds the lists the gate_up phase
  // built from the same router ids.
  constexpr bool kListsBuilt = PHASE == kPhaseDown;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int IPE = EPI == EPI_ACT ? p.inter / 8 : p.N / 16;  // items per expert
  const uint16_t* A16 = (const uint16_t*)p.A;
  uint16_t* C = (uint16_t*)p.C;
  uint8_t* ring = smem + w * WAVE_RING;

  MSTAR_TL(0);
  // ---- prologue 1: per-expert counts and the active-expert mask.
  int my_e[SPT], my_pos[SPT];
  // Layer gate_up phase: the last wave (the one with the fewest items)
  // claims the own range (0 -> 1) once its router ids have arrived, so that
  // no wait of the prologue waits for it; its answer is read after the
  // wave's first weight chunk.
  constexpr int CW = NWV - 1;
  int own_old = 1;
  if constexpr (!kListsBuilt) {
    // All of a thread's id loads in flight at once (one round trip): buffer
    // loads, which return 0 past the ids without a branch around them.
    const bool i64 = p.ids_dtype == kI64;
    const auto rs_ids = make_rsrc(p.topk_ids, (uint32_t)(p.M * (i64 ? 8 : 4)));
    int lo[SPT], hi[SPT];
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const uint32_t i = (uint32_t)(tid + j * NTH);
      lo[j] = __builtin_amdgcn_raw_buffer_load_b32(rs_ids, i64 ? i * 8 : i * 4, 0, 0);
      hi[j] = i64 ? __builtin_amdgcn_raw_buffer_load_b32(rs_ids, i * 8 + 4, 0, 0) : 0;
    }
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const int i = tid + j * NTH;
      // Out-of-range ids (negative or >= E, or a high word set) are skipped (.cu:44-46).
      const bool ok = i < p.M && lo[j] >= 0 && lo[j] < E && (i64 ? hi[j] == 0 : true);
      my_e[j] = ok ? lo[j] : -1;
      my_pos[j] = 0;
    }
    if constexpr (PHASE == kPhaseGate) {
      if (own && w == CW && lane == 0 && !(ls.mode == kLayerTestNoOwnClaim && (blockIdx.x & 1))) {
        own_old = 0;
        __hip_atomic_compare_exchange_strong(ls.claim + wg * kClaimStride, &own_old, 1, __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    for (int e = tid; e < E; e += NTH) sCnt[e] = 0;
    if (tid < 32) sMask[tid] = 0;
    MSTAR_TL(1);
    lds_sync();
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const int e = my_e[j];
      if (e >= 0) {
        my_pos[j] = atomicAdd(&sCnt[e], 1);
        atomicOr(&sMask[e >> 5], 1u << (e & 31));
      }
    }
    lds_sync();
  }
  // Active experts: prefix popcounts of the mask words (lane i: word i).
  MSTAR_TL(2);
  const uint32_t mword = lane < 32 ? sMask[lane] : 0u;
  const int wincl = wave_incl_scan(__builtin_popcount(mword));
  const int n_act = wave_last(wincl);
  const int total = n_act * IPE;
  const int T = (total + nwg - 1) / nwg;
  int i0 = wg * T;
  int i1 = i0 + T < total ? i0 + T : total;
  // Without work a workgroup is done, except that the gate_up phase of the
  // layer kernel still builds the lists for its down phase.
  if (i0 >= i1 && PHASE != kPhaseGate) return;
  auto active_expert = [&](int a) -> int {  // the a-th active expert (wave-uniform a)
    const uint64_t past = __ballot(wincl > a);
    const int word = __builtin_ctzll(past);
    uint32_t m = (uint32_t)__shfl((int)mword, word, 64);
    int skip = a - (__shfl(wincl, word, 64) - __builtin_popcount(m));
    for (; skip > 0; --skip) m &= m - 1u;
    return word * 32 + __builtin_ctz(m);
  };

  // ---- weight DMA of (item, chunk) into ring slot `slot`.  DMA lane geometry:
  // rows r8 and 8 + r8 of the item, physical chunk pc = logical pc ^ r8.
  const int r8 = lane >> 3;
  const uint32_t lc16 = (uint32_t)(((lane & 7) ^ r8) * 16);
  // int4 rows (see dma_rows): the source piece of lane l in instructions 0
  // and 1, and the byte distance from row r8 to row 8 + r8.
  const uint32_t w4_lc0 = (uint32_t)(((lane & 7) ^ w4_swz(r8)) * 16);
  const uint32_t w4_lc1 = (uint32_t)(((lane & 7) ^ w4_swz(8 + r8)) * 16);
  const int64_t w4_q1 = (int64_t)(EPI == EPI_ACT ? p.inter : 8) * p.ldb * 4;
  const Int4BiasConsts w4k = int4_bias_consts();
  auto dma_rows = [&](int e, int g, const uint8_t*& s0, const uint8_t*& s1) {
    if constexpr (W4) {
      // A chunk's two K-steps are one 128-byte line of each row.  DMA
      // instruction q moves item rows 8q .. 8q+7: lane l row 8q + l / 8,
      // physical piece l % 8 holding logical piece (l % 8) ^ w4_swz(row)
      // (logical piece = 4 * K-step + 16-byte piece of the step's 64 bytes).
      // s0 is row r8 of instruction 0; instruction 1's row is w4_q1 bytes
      // further.  Lanes 0-15 also fetch item row l's scales (s1).  Item rows
      // 0-7 are gate rows and 8-15 the matching up rows (EPI_ACT).
      auto row_of = [&](int rr) -> int {
        if constexpr (EPI == EPI_ACT) return rr < 8 ? g * 8 + rr : p.inter + g * 8 + rr - 8;
        else return g * 16 + rr;
      };
      const uint8_t* Be = (const uint8_t*)p.B + (int64_t)e * p.b_estride * 4;  // int32 words
      s0 = Be + (int64_t)row_of(r8) * p.ldb * 4;
      s1 = (const uint8_t*)((const uint16_t*)p.b_scale + (int64_t)e * p.bs_estride +
                            (int64_t)row_of((lane / W4_PR) & 15) * p.bs_ld) + (lane % W4_PR) * 4;
      return;
    }
    const uint8_t* Be = (const uint8_t*)p.B + (int64_t)e * p.b_estride;
    int row0, row1;
    if constexpr (EPI == EPI_ACT) {
      row0 = g * 8 + r8;
      row1 = p.inter + g * 8 + r8;
    } else {
      row0 = g * 16 + r8;
      row1 = g * 16 + 8 + r8;
    }
    s0 = Be + (int64_t)row0 * p.ldb + lc16;
    s1 = Be + (int64_t)row1 * p.ldb + lc16;
  };
  auto dma = [&](const uint8_t* s0, const uint8_t* s1, int c, int slot) {
    uint8_t* dst = ring + slot * SLOT;
    if constexpr (W4) {
#pragma unroll
      for (int h = 0; h < KC / 2; ++h) {  // line h of the chunk: rows 0-7, then 8-15
        const int64_t lo = (int64_t)(c * (KC / 2) + h) * 128;
        __builtin_amdgcn_global_load_lds((const void*)(s0 + lo + w4_lc0), (lds_void_ptr)(dst + 2 * h * 1024),
                                         16, 0, kDmaAux);
        __builtin_amdgcn_global_load_lds((const void*)(s0 + w4_q1 + lo + w4_lc1),
                                         (lds_void_ptr)(dst + (2 * h + 1) * 1024), 16, 0, kDmaAux);
      }
      if (lane < 16 * W4_PR)  // piece lane % W4_PR of row lane / W4_PR's scales of the chunk
        __builtin_amdgcn_global_load_lds((const void*)(s1 + c * KC * 2), (lds_void_ptr)(dst + KC * 1024),
                                         4, 0, 0);
      return;
    }
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
      __builtin_amdgcn_global_load_lds((const void*)(s0 + (c * KC + kk) * 128),
                                       (lds_void_ptr)(dst + kk * 2048), 16, 0, kDmaAux);
      __builtin_amdgcn_global_load_lds((const void*)(s1 + (c * KC + kk) * 128),
                                       (lds_void_ptr)(dst + kk * 2048 + 1024), 16, 0, kDmaAux);
    }
  };

  // ---- prefetch: waves that do not stage start their first item's weights
  // now; lds_sync leaves the DMA in flight through the rest of the prologue.
  const int it_first = i0 + w;
  const bool prefetched = w >= SW && it_first < i1;
  if (prefetched) {
    const int a = it_first / IPE;
    const uint8_t *s0, *s1;
    dma_rows(active_expert(a), it_first - a * IPE, s0, s1);
#pragma unroll
    for (int c = 0; c < RING - 1; ++c)
      if (c < CH) dma(s0, s1, c, c);
  }

  // ---- prologue 2: offsets, active list, slot lists.
  if constexpr (!kListsBuilt) {
    if (w == 0) {
      int run = 0;
      for (int e0 = 0; e0 < E; e0 += 64) {
        const int e = e0 + lane;
        const int c = e < E ? sCnt[e] : 0;
        const int incl = wave_incl_scan(c);
        if (e < E) sOff[e] = run + incl - c;
        run += wave_last(incl);
      }
      int n = 0;
      for (int e0 = 0; e0 < E; e0 += 64) {
        const int e = e0 + lane;
        const bool act = e < E && sCnt[e] > 0;
        const uint64_t b = __ballot(act);
        if (act) sAct[n + __builtin_popcountll(b & ((1ull << lane) - 1ull))] = e;
        n += __builtin_popcountll(b);
      }
    }
    if (PHASE == kPhaseGate && w == 0 && lane == 0) sFlags[kFlagOwn] = 1;  // until told otherwise
    lds_sync();
#pragma unroll
    for (int j = 0; j < SPT; ++j)
      if (my_e[j] >= 0) sList[sOff[my_e[j]] + my_pos[j]] = tid + j * NTH;
    lds_sync();
  }
  // Layer gate_up phase, own range: if another workgroup took the range
  // first (the answer to the last wave's claim, published after its first
  // chunk), sFlags[kFlagOwn] is cleared, which every wave checks before each
  // unit: a late start stops within a unit; rows written meanwhile get the
  // same values from the taker, and only the taker reports them.  At the end
  // of its items the last wave claims the other gate_up ranges its down
  // range waits on (0 -> 2): by then every resident workgroup has claimed
  // its own.
  bool own_pending = PHASE == kPhaseGate && own;
  // The answers -> sFlags: whether the own range is this workgroup's, and
  // the ranges it took.
  auto claim_dependencies = [&]() {
    if constexpr (PHASE == kPhaseGate) {
      if (!own || w != CW) return;
      int dep_lo, dep_hi;
      layer_dependencies(n_act, IPE, ls.down_ipe, nwg, wg, &dep_lo, &dep_hi);
      int nst = 0;
      for (int qb = dep_lo; qb <= dep_hi && nst < kMaxSteals; qb += 64) {
        const int q = qb + lane;
        int old = 1;
        if (q <= dep_hi) {  // the own range too: it fails unless nobody has claimed it
          old = 0;
          __hip_atomic_compare_exchange_strong(ls.claim + q * kClaimStride, &old, 2, __ATOMIC_RELAXED,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const uint64_t won = __ballot(old == 0);
        const int before = __builtin_popcountll(won & ((1ull << lane) - 1ull));
        if (old == 0 && nst + before < kMaxSteals) sFlags[kFlagSteal + nst + before] = q;
        nst += __builtin_popcountll(won);
      }
      if (lane == 0) {
        const int z = sFlags[kFlagOwn] - 1;  // 0, or -1 if already cleared (own_old != 0 then)
        sFlags[kFlagOwn] = (own_old | z) == 0;
        sFlags[kFlagStealN] = nst < kMaxSteals ? nst : kMaxSteals;
      }
    }
  };
  // The layer's gate_up phase runs its own range, then the ranges it took
  // over (passes).
  bool run_pass = PHASE != kPhaseGate || i0 < i1;
  int a_first = i0 / IPE, a_last = (i1 - 1) / IPE;
  MSTAR_TL(3);

  // ---- staging (waves < SW): `nrows` rows; row j reads A row arow_of(j).
  // The staging waves hold no prefetched weights, so their loads are all in
  // flight at once and one wait covers them.
  constexpr int ST = SW * 64;
  auto stage_copy_q16 = [&](int nrows, auto arow_of) {
    if constexpr (KS % 4 == 0) {
      // LDS-DMA: 1 KB (64 lanes x 16 bytes) of one row per instruction.
      constexpr int CPR = KS / 4;  // 1 KB pieces per row
      for (int pc = w; pc < nrows * CPR; pc += SW) {
        const int r = pc / CPR, c = pc - r * CPR;
        __builtin_amdgcn_global_load_lds((const void*)(A16 + (int64_t)arow_of(r) * p.lda + c * 512 + lane * 8),
                                         (lds_void_ptr)(sRows + r * PITCH + c * 1024), 16, 0, 0);
      }
    } else {
      constexpr int PPR = KS * 16;  // 16-byte pieces per row
      const int pieces = nrows * PPR;
      for (int base = 0; base < pieces; base += ST * 8) {
        v4i v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int pc = base + j * ST + tid;
          const int r = pc / PPR, c = pc - r * PPR;
          v[j] = pc < pieces ? *(const v4i*)(A16 + (int64_t)arow_of(r) * p.lda + c * 8) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int pc = base + j * ST + tid;
          const int r = pc / PPR, c = pc - r * PPR;
          if (pc < pieces) *(v4i*)(sRows + r * PITCH + c * 16) = v[j];
        }
      }
    }
    if constexpr (!W4)  // token block scales
      for (int i = tid; i < nrows * KS; i += ST) {
        const int r = i / KS, ks = i - r * KS;
        sSc[i] = p.a_scale[(int64_t)arow_of(r) * p.ld_as + ks];
      }
    wait_vmcnt<0>();
  };
  auto stage_quant = [&](int nrows, auto arow_of) {
    constexpr int B = 8;
    const int groups = nrows * KS;
    for (int g0 = 0; g0 < groups; g0 += (ST / 16) * B) {
      v4i raw[B];
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const int gq = g0 + j * (ST / 16) + (tid >> 4), sub = tid & 15;
        const bool live = gq < groups;
        const int r = live ? gq / KS : 0, ks = live ? gq - (gq / KS) * KS : 0;
        raw[j] = live ? load_rows16<PHASE == kPhaseDown>(A16 + (int64_t)arow_of(r) * p.lda + ks * 128 + sub * 8)
                      : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const int gq = g0 + j * (ST / 16) + (tid >> 4), sub = tid & 15;
        const bool live = gq < groups;
        const int r = live ? gq / KS : 0, ks = live ? gq - (gq / KS) * KS : 0;
        float sc;
        const int2 codes = quant_group8<kBF16>(raw[j], sc);
        if (live) {
          *(v4i*)(sRows + r * PITCH + ks * 256 + sub * 16) = fp8x8_to_bf16x8_bits(codes.x, codes.y);
          if (sub == 0) sSc[r * KS + ks] = sc;
        }
      }
    }
  };

  // W4: token rows as bf16, each group of 8 reordered to 0, 4, 1, 5, 2, 6,
  // 3, 7, and the fp32 sum of each 128-element block into sSc.
  auto stage_w4 = [&](int nrows, auto arow_of) {
    constexpr int B = 8;
    const int groups = nrows * KS;
    for (int g0 = 0; g0 < groups; g0 += (ST / 16) * B) {
      v4i raw[B];
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const int gq = g0 + j * (ST / 16) + (tid >> 4), sub = tid & 15;
        const bool live = gq < groups;
        const int r = live ? gq / KS : 0, ks = live ? gq - (gq / KS) * KS : 0;
        raw[j] = live ? load_rows16<PHASE == kPhaseDown>(A16 + (int64_t)arow_of(r) * p.lda + ks * 128 + sub * 8)
                      : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const int gq = g0 + j * (ST / 16) + (tid >> 4), sub = tid & 15;
        const bool live = gq < groups;
        const int r = live ? gq / KS : 0, ks = live ? gq - (gq / KS) * KS : 0;
        const uint32_t d0 = raw[j][0], d1 = raw[j][1], d2 = raw[j][2], d3 = raw[j][3];
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t d = (uint32_t)raw[j][i];
          sum += bf16_bits_to_f32((uint16_t)(d & 0xffffu)) + bf16_bits_to_f32((uint16_t)(d >> 16));
        }
        sum = row_fsum16(sum);  // the 16 lanes of a block are one DPP row
        if (live) {
          const v4i o = v4i{(int)((d0 & 0xffffu) | (d2 << 16)), (int)((d0 >> 16) | (d2 & 0xffff0000u)),
                            (int)((d1 & 0xffffu) | (d3 << 16)), (int)((d1 >> 16) | (d3 & 0xffff0000u))};
          *(v4i*)(sRows + r * PITCH + ks * 256 + sub * 16) = o;
          if (sub == 0) sSc[r * KS + ks] = sum;
        }
      }
    }
    wait_vmcnt<0>();
  };

  // ---- the wave's units in a window: (item, pass of up to 16 rows).  A
  // cursor walks them; the issue cursor runs kCuRing - 1 chunks ahead of
  // the compute cursor.
  struct Cur {
    int it, r0, c;  // item, first row of the pass, chunk
  };
  int wa0 = 0, wa1 = -1, wr0 = 0, wr1 = 0;
  auto item_rows = [&](int it, int& rb, int& re) -> bool {  // row range of `it` in the window
    const int a = it / IPE;
    if (a < wa0 || a > wa1) return false;
    const int cnt = __builtin_amdgcn_readfirstlane(sCnt[sAct[a]]);
    rb = a == wa0 ? wr0 : 0;
    re = (a == wa0 && wr1 < cnt) ? wr1 : cnt;
    return rb < re;
  };
  auto first_unit = [&](int it, Cur& cu) -> bool {  // first unit at or after item `it`
    for (; it < i1; it += NWV) {
      int rb, re;
      if (item_rows(it, rb, re)) {
        cu = Cur{it, rb, 0};
        return true;
      }
    }
    return false;
  };
  auto advance = [&](Cur& cu) -> bool {  // next chunk
    if (++cu.c < CH) return true;
    int rb, re;
    item_rows(cu.it, rb, re);
    if (cu.r0 + 16 < re) {
      cu.r0 += 16;
      cu.c = 0;
      return true;
    }
    return first_unit(cu.it + NWV, cu);
  };

  bool use_prefetch = prefetched;
  bool poison = false;  // down phase: the window's wait gave up (NaN rows)
  int pass = 0;  // gate_up passes: the own range, then ranges taken over
  auto run_window = [&](int lbase) {
    Cur ic, cc;  // issue / compute cursors
    bool ihas = first_unit(i0 + w, ic);
    if (!ihas) {
      if (use_prefetch) wait_vmcnt<0>();  // the prefetch targeted a later window: retire it
      use_prefetch = false;
      return;
    }
    cc = ic;
    // Issue the first RING - 1 chunks (or adopt the prefetch).
    int ahead = 0;      // chunks issued beyond the compute cursor
    int islot = 0;      // ring slot of the next issue
    const uint8_t *is0, *is1;
    int icur_it = -1, icur_r0 = -1;
    auto issue_next = [&]() {
      if (ic.it != icur_it || ic.r0 != icur_r0) {
        const int a = ic.it / IPE;
        dma_rows(sAct[a], ic.it - a * IPE, is0, is1);
        icur_it = ic.it;
        icur_r0 = ic.r0;
      }
      dma(is0, is1, ic.c, islot);
      islot = islot + 1 == RING ? 0 : islot + 1;
      ++ahead;
      ihas = advance(ic);
    };
    const bool adopt = use_prefetch && ic.it == it_first && ic.c == 0;
    if (use_prefetch && !adopt) wait_vmcnt<0>();  // retire a prefetch this window does not use
    use_prefetch = false;
    for (int n = 0; n < RING - 1 && ihas; ++n) {
      if (adopt) {  // already in flight
        if (ic.it != icur_it || ic.r0 != icur_r0) {
          const int a = ic.it / IPE;
          dma_rows(sAct[a], ic.it - a * IPE, is0, is1);
          icur_it = ic.it;
          icur_r0 = ic.r0;
        }
        if (ic.it != it_first || ic.r0 != cc.r0) break;  // the prefetch covered only the first unit
        islot = islot + 1 == RING ? 0 : islot + 1;
        ++ahead;
        ihas = advance(ic);
      } else {
        issue_next();
      }
    }
    int cslot = 0;
    while (true) {
      // ---- unit set-up (compute side)
      if constexpr (PHASE == kPhaseGate) {
        if (pass == 0 && !__builtin_amdgcn_readfirstlane(sFlags[kFlagOwn])) return;  // the range was taken
      }
      const int a = cc.it / IPE, g = cc.it - a * IPE;
      const int e = __builtin_amdgcn_readfirstlane(sAct[a]);
      const int off = __builtin_amdgcn_readfirstlane(sOff[e]);
      int rb, re;
      item_rows(cc.it, rb, re);
      const int rows = re - cc.r0 < 16 ? re - cc.r0 : 16;
      const bool tok_ok = l16 < rows;
      const int li = off + cc.r0 + (tok_ok ? l16 : 0);
      const int slot_id = sList[li];
      const int lrow = li - lbase;
      const uint8_t* trow = sRows + lrow * PITCH + lg * 64;
      const float* tsc = sSc + lrow * KS;
      // Element offsets of the weight-block scale rows of this unit's outputs
      // (gate block for lanes lg < 2, up block above).
      int blk_lo, blk_hi;
      if constexpr (EPI == EPI_ACT) {
        blk_lo = (g * 8) / 128;
        blk_hi = (p.inter + g * 8) / 128;
      } else {
        blk_lo = blk_hi = (g * 16) / 128;
      }
      const int so_lo = (int)(e * p.bs_estride) + blk_lo * (int)p.bs_ld;
      const int so_hi = (int)(e * p.bs_estride) + blk_hi * (int)p.bs_ld;
      // Read-only for the whole launch: reading it through the constant
      // address space lets the compiler use scalar loads.
      typedef const __attribute__((address_space(4))) float* const_fptr;
      const const_fptr bsc = (const_fptr)p.b_scale;
      v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
      const int unit_it = cc.it, unit_r0 = cc.r0;
      // ---- chunks of the unit
      while (true) {
        while (ihas && ahead < RING) issue_next();
        // Wait for this chunk's DMA, leaving the later ones in flight (two
        // fewer, for the epilogue store / routed-weight load that may sit
        // between them: over-waiting is safe).
        wait_leaving_chunks<DPC, RING>(ahead);
        if constexpr (PHASE == kPhaseGate) {
          if (w == CW && own_pending) {  // the claim's answer: older than this chunk's DMA
            own_pending = false;
            // z is 0 (sFlags[kFlagOwn] is still 1: this wave is its only
            // writer); folding it in keeps the compiler from testing the
            // answer -- and so waiting for it -- right after the claim.
            const int z = sFlags[kFlagOwn] - 1;
            if (lane == 0 && (own_old | z) != 0) sFlags[kFlagOwn] = 0;
          }
        }
        const uint8_t* wslot = ring + cslot * SLOT;
        // Wave-uniform, so the weight-scale reads below are scalar loads (a
        // vector load here would make the compiler drain the DMA queue).
        const int c = __builtin_amdgcn_readfirstlane(cc.c);
        if constexpr (W4) {
          // Scales of rows 4 lg .. +3 (the rows this lane's results belong
          // to) for the chunk's K-steps: 8 KC contiguous bytes.
          v4i sc4[W4_PR];
#pragma unroll
          for (int h = 0; h < W4_PR; ++h) sc4[h] = *(const v4i*)(wslot + KC * 1024 + lg * 8 * KC + h * 16);
#pragma unroll
          for (int kk = 0; kk < KC; ++kk) {
            const int ks = c * KC + kk;
            const v4i wq = *(const v4i*)(wslot + ((kk >> 1) * 2 + (l16 >> 3)) * 1024 + (l16 & 7) * 128 +
                                         ((((kk & 1) * 4 + lg) ^ w4_swz(l16)) << 4));
            v4f t = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < 4; ++m)
              t = mfma_bf16_16x16x32(int4x8_bias128((uint32_t)wq[m], w4k), *(const v8s*)(trow + ks * 256 + m * 16), t);
            // sum (u - 8) x = sum (u + 128) x - 136 sum x, then the row's scale
            // (q * s is exact in bf16, so scaling after the sum is the
            // bf16(q * s) weight's product).
            const float bias = 136.f * tsc[ks];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              // Row r's scale of K-step kk: half kk % 2 of dword r W4_PR + kk / 2.
              const int dw = r * W4_PR + (kk >> 1);
              const uint32_t two = (uint32_t)sc4[dw >> 2][dw & 3];
              const float sr = bf16_bits_to_f32((uint16_t)((kk & 1) == 0 ? two & 0xffffu : two >> 16));
              acc[r] += (t[r] - bias) * sr;
            }
          }
        } else {
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) {
          const int ks = c * KC + kk;
          const uint8_t* wrow = wslot + kk * 2048 + l16 * 128;
          const int sw = l16 & 7;
          const v4i wlo = *(const v4i*)(wrow + (((2 * lg) ^ sw) << 4));
          const v4i whi = *(const v4i*)(wrow + (((2 * lg + 1) ^ sw) << 4));
          // Scalar loads: the indices are wave-uniform by construction.
          const float slo = bsc[__builtin_amdgcn_readfirstlane(so_lo + ks)];
          const float shi = bsc[__builtin_amdgcn_readfirstlane(so_hi + ks)];
          const float f = tsc[ks] * (lg < 2 ? slo : shi);
          v4f t = v4f{0.f, 0.f, 0.f, 0.f};
          t = mfma_bf16_16x16x32(fp8x8_to_bf16x8(wlo[0], wlo[1]), *(const v8s*)(trow + ks * 256), t);
          t = mfma_bf16_16x16x32(fp8x8_to_bf16x8(wlo[2], wlo[3]), *(const v8s*)(trow + ks * 256 + 16), t);
          t = mfma_bf16_16x16x32(fp8x8_to_bf16x8(whi[0], whi[1]), *(const v8s*)(trow + ks * 256 + 32), t);
          t = mfma_bf16_16x16x32(fp8x8_to_bf16x8(whi[2], whi[3]), *(const v8s*)(trow + ks * 256 + 48), t);
          acc += t * f;
        }
        }
        cslot = cslot + 1 == RING ? 0 : cslot + 1;
        --ahead;
        const bool more = advance(cc);
        if (!more || cc.it != unit_it || cc.r0 != unit_r0) {
          // ---- epilogue of the unit: lane (l16, lg) holds weight rows 4 lg + r for token l16.
          if constexpr (EPI == EPI_ACT) {
            // Gate rows 0-7 sit in lanes lg 0-1, the matching up rows 32 lanes up.
            float up[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) up[r] = __shfl_xor(acc[r], 32, 64);
            if (lg < 2 && tok_ok) {
              uint32_t pk[2];
#pragma unroll
              for (int h = 0; h < 2; ++h) {
                uint32_t two = 0;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                  const int r = 2 * h + q;
                  const float gg = round_bf16(acc[r]);
                  const float u = round_bf16(up[r]);
                  const float av = round_bf16(p.activation == 0 ? act_f32<0>(gg) : act_f32<1>(gg));
                  two |= (uint32_t)f32_to_bf16_bits(av * u) << (16 * q);
                }
                pk[h] = two;
              }
              uint16_t* dst = C + (int64_t)slot_id * p.ldc + g * 8 + 4 * lg;
              if constexpr (PHASE == kPhaseGate)  // read by other XCDs' down phases
                __hip_atomic_store((uint64_t*)dst, (uint64_t)pk[0] | ((uint64_t)pk[1] << 32), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
              else
                *(uint2*)dst = make_uint2(pk[0], pk[1]);
            }
          } else {
            if (tok_ok) {
              const float rw = p.mul_routed ? sRw[lrow] : 1.f;
              uint32_t lo = (uint32_t)f32_to_bf16_bits(acc[0] * rw) |
                            ((uint32_t)f32_to_bf16_bits(acc[1] * rw) << 16);
              uint32_t hi = (uint32_t)f32_to_bf16_bits(acc[2] * rw) |
                            ((uint32_t)f32_to_bf16_bits(acc[3] * rw) << 16);
              if (PHASE == kPhaseDown && poison) lo = hi = 0x7fc07fc0u;  // bf16 NaN: the wait gave up
              *(uint2*)(C + (int64_t)slot_id * p.ldc + g * 16 + 4 * lg) = make_uint2(lo, hi);
            }
          }
          if (!more) return;
          break;
        }
      }
    }
  };

  for (;; ++pass) {
  // Windows over the CU's experts: as many whole experts as fit in `cap`
  // rows, or `cap` rows of one larger expert.  Usually a single window.
  int a = run_pass ? a_first : a_last + 1, r = 0;
  bool first_window = true;
  while (a <= a_last) {
    wa0 = a;
    wr0 = r;
    wa1 = a;
    wr1 = 0x7fffffff;
    int nrows;
    const int rem = sCnt[sAct[a]] - r;
    if (rem > cap) {
      nrows = cap;
      wr1 = r + cap;
      r += cap;
    } else {
      nrows = rem;
      ++a;
      r = 0;
      while (a <= a_last && nrows + sCnt[sAct[a]] <= cap) {
        nrows += sCnt[sAct[a]];
        wa1 = a;
        ++a;
      }
    }
    const int lbase = sOff[sAct[wa0]] + wr0;  // list index of staged row 0
    if (!first_window) lds_sync();             // every wave is done with the previous window
    first_window = false;
    if constexpr (PHASE == kPhaseDown) {
      // Wait until the gate_up phases reported every row of the window's
      // experts (one wave polls, a lane per expert, about once a
      // microsecond: every poll is a memory request that competes with the
      // weight streams), then the staging waves acquire their stores.
      if (w == 0) {
        bool gave_up = false;
        for (int aa = wa0 + lane; aa <= wa1; aa += 64) {
          const int e = sAct[aa];
          const int target = ls.gate_ipe * sCnt[e];
          const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
          while (__hip_atomic_load(ls.done + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (ls.mode == kLayerTestGiveUp || __builtin_amdgcn_s_memrealtime() - t0 > kLayerWaitTicks) {
              gave_up = true;
              break;
            }
            __builtin_amdgcn_s_sleep(32);
          }
          if (ls.mode == kLayerTestGiveUp) gave_up = true;
        }
        const bool any = __ballot(gave_up) != 0;
        if (lane == 0) {
          sFlags[kFlagPoison] = any;
          if (any) {
            __hip_atomic_store(ls.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(&g_layer_wait_failures, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
      lds_sync();  // the staging reads the rows as agent-scope atomics (load_rows16)
      poison = __builtin_amdgcn_readfirstlane(sFlags[kFlagPoison]) != 0;
    }
    if (w < SW) {
      const auto arow_of = [&](int j) { return sList[lbase + j] / p.top_k; };
      if constexpr (STAGE == STAGE_Q16) stage_copy_q16(nrows, arow_of);
      else if constexpr (STAGE == STAGE_W4) stage_w4(nrows, arow_of);
      else stage_quant(nrows, arow_of);
      if (EPI != EPI_ACT && p.mul_routed)
        for (int j = tid; j < nrows; j += ST)
          sRw[j] = load_weight_any(p.topk_w, p.topk_w_dtype, sList[lbase + j]);
    }
    lds_sync();
    MSTAR_TL(4);
    run_window(lbase);
    MSTAR_TL(5);
  }
  if (pass == 0) claim_dependencies();
  wait_vmcnt<0>();  // no DMA outlives the kernel
  MSTAR_TL(7);
  if constexpr (PHASE != kPhaseGate) {
    break;
  } else {
    // Report this range's (item, row) pairs per expert once every wave's
    // stores are complete (the wait above): one lane per expert adds
    // (items of the expert in [i0, i1)) x (its rows).  The activation rows
    // were stored as agent-scope atomics, which are coherent across XCDs
    // without the L2 write-back an agent-scope release fence costs.
    lds_sync();  // also: the list of ranges taken over is written
    // Only the range's claimant reports it.
    if (w == 0 && run_pass && (pass > 0 || sFlags[kFlagOwn])) {
      for (int a = a_first + lane; a <= a_last; a += 64) {
        const int lo = i0 > a * IPE ? i0 : a * IPE;
        const int hi = i1 < (a + 1) * IPE ? i1 : (a + 1) * IPE;
        const int e = sAct[a];
        __hip_atomic_fetch_add(ls.done + e, (hi - lo) * sCnt[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // Next pass: a range taken over (claimed, with items, by construction).
    if (!own || pass >= __builtin_amdgcn_readfirstlane(sFlags[kFlagStealN])) break;
    const int q = __builtin_amdgcn_readfirstlane(sFlags[kFlagSteal + pass]);
    i0 = q * T;
    i1 = i0 + T < total ? i0 + T : total;
    a_first = i0 / IPE;
    a_last = (i1 - 1) / IPE;
    run_pass = i0 < i1;
    use_prefetch = false;
  }
  }
}

template <int EPI, int KS, int STAGE>
__global__ __launch_bounds__(STAGE == STAGE_W4 ? kCuThreadsW4 : kCuThreads) void stream_fp8_cu_kernel(
    GemmArgs p, int cap) {
  stream_cu_body<EPI, KS, STAGE>(p, cap, blockIdx.x, gridDim.x, LayerSync{});
}

// Range of workgroup b: consecutive ranges go to workgroups of one XCD
// (workgroups are dealt to the 8 XCDs round-robin), so the gate_up ranges
// an expert's down work waits on ran on the same XCD.
__device__ __forceinline__ int xcd_range(int b, int nwg) {
  return nwg % 8 == 0 ? (b % 8) * (nwg / 8) + b / 8 : b;
}

// The decode layer's two streaming GEMMs in one launch: each workgroup
// runs its gate_up range (FP8: bf16-widened FP8 token rows from the routing
// launch; W4: bf16 hidden rows -> bf16 SiLU-and-mul rows), then the gate_up
// ranges it stole (those its down range waits on that nobody had claimed),
// then its down range, staging an expert's rows once the gate_up work that
// covers the expert is reported (LayerSync).  No gate_up work ever waits,
// and every range a down-phase wait depends on is claimed by a running
// workgroup before the wait begins, so the waits end whatever subset of
// the workgroups is resident at a time.
template <int KS1, int KS2, bool W4>
__global__ __launch_bounds__(W4 ? kCuThreadsW4 : kCuThreads) void stream_layer_kernel(GemmArgs g1, GemmArgs g2,
                                                                                   int cap1, int cap2,
                                                                                   LayerSync ls) {
  const int r = xcd_range(blockIdx.x, gridDim.x);
  stream_cu_body<EPI_ACT, KS1, W4 ? STAGE_W4 : STAGE_Q16, kPhaseGate>(g1, cap1, r, gridDim.x, ls);
  __syncthreads();  // every wave is done with the gate_up phase's LDS
  stream_cu_body<EPI_STORE, KS2, W4 ? STAGE_W4 : STAGE_H16, kPhaseDown>(g2, cap2, r, gridDim.x, ls);
}


template <int EPI, int KS, bool EXACT, bool AQ>
static int run_stream_fp8(const GemmArgs& a, hipStream_t stream) {
  constexpr int K = KS * 128;
  const size_t shmem = (size_t)kStreamRows * (K + 16) + (size_t)KS * kStreamRows * 4 +
                       kStreamRows * 4 + (size_t)a.num_experts * 3 * 4 +
                       (a.topk_ids ? (size_t)a.M * 4 : 0);
  auto kern = stream_fp8_kernel<EPI, KS, EXACT, AQ>;
  const int st = ensure_dynamic_lds((const void*)kern, shmem, "stream_fp8");
  if (st != kOk) return st;
  // Persistent: as many workgroups as can be resident at this LDS size (at
  // most four per CU).
  int occ = occupancy_per_cu((const void*)kern, 256, shmem);
  if (occ > kStreamWgPerCu) occ = kStreamWgPerCu;
  const int cus = device_cu_count();
  if (occ <= 0 || cus <= 0) return kLaunchError;
  const int grid = occ * cus;
  kern<<<dim3(grid), dim3(256), shmem, stream>>>(a);
  return launch_status("stream_fp8");
}

template <int EPI, int KS, int STAGE>
static int run_stream_fp8_cu(const GemmArgs& a, int cap, size_t shmem, hipStream_t stream) {
  auto kern = stream_fp8_cu_kernel<EPI, KS, STAGE>;
  const int st = ensure_dynamic_lds((const void*)kern, shmem, "stream_fp8_cu");
  if (st != kOk) return st;
  const int cus = device_cu_count();
  if (cus <= 0) return kLaunchError;
  kern<<<dim3(cus), dim3(STAGE == STAGE_W4 ? kCuThreadsW4 : kCuThreads), shmem, stream>>>(a, cap);
  return launch_status("stream_fp8_cu");
}

// The CU-resident kernel for (exact, router-ids mode), or false if the shape
// does not fit it.
template <int KS>
static bool try_stream_fp8_cu(const GemmArgs& a, int epi, hipStream_t stream, int* status,
                              bool int4 = false) {
  const size_t per_row = (size_t)cu_pitch<KS>() + (KS + 1) * 4;
  if (a.a_scale && !a.a_q16) return false;  // e4m3fn rows: the LDS-staged kernel
  if (int4 && (KS % 2 != 0 || a.a_scale)) return false;
  // Rows staged per window: as many as the LDS budget allows.
  // 1 KB stays free for the kernel's static LDS.
  const size_t fixed = (int4 ? cu_sc_off<KS, true>(a.num_experts, a.M) : cu_sc_off<KS>(a.num_experts, a.M)) +
                       16 + 1024;
  if (fixed + 4 * per_row > kCuLdsMax) return false;  // windows need a few rows
  int cap = (int)((kCuLdsMax - fixed) / per_row);
  if (cap > 1024) cap = 1024;
  const size_t shmem = (int4 ? cu_rows_off<KS, true>(a.num_experts, a.M, cap)
                             : cu_rows_off<KS>(a.num_experts, a.M, cap)) + (size_t)cap * cu_pitch<KS>();
  if constexpr (KS % 2 == 0) {
    if (int4) {
      *status = epi == EPI_ACT ? run_stream_fp8_cu<EPI_ACT, KS, STAGE_W4>(a, cap, shmem, stream)
                               : run_stream_fp8_cu<EPI_STORE, KS, STAGE_W4>(a, cap, shmem, stream);
      return true;
    }
  }
  if (a.a_q16)
    *status = epi == EPI_ACT ? run_stream_fp8_cu<EPI_ACT, KS, STAGE_Q16>(a, cap, shmem, stream)
                             : run_stream_fp8_cu<EPI_STORE, KS, STAGE_Q16>(a, cap, shmem, stream);
  else
    *status = epi == EPI_ACT ? run_stream_fp8_cu<EPI_ACT, KS, STAGE_H16>(a, cap, shmem, stream)
                             : run_stream_fp8_cu<EPI_STORE, KS, STAGE_H16>(a, cap, shmem, stream);
  return true;
}

// Rows a window of the CU-resident kernel stages, and its dynamic LDS.
template <int KS, bool W4>
static bool cu_window(const GemmArgs& a, size_t lists_at, int* cap_out, size_t* shmem_out) {
  const size_t per_row = (size_t)cu_pitch<KS>() + (KS + 1) * 4;
  const size_t fixed = cu_sc_off<KS, W4>(a.num_experts, a.M, lists_at) + 16 + 1024;
  if (fixed + 4 * per_row > kCuLdsMax) return false;
  int cap = (int)((kCuLdsMax - fixed) / per_row);
  if (cap > 1024) cap = 1024;
  *cap_out = cap;
  *shmem_out = cu_rows_off<KS, W4>(a.num_experts, a.M, cap, lists_at) + (size_t)cap * cu_pitch<KS>();
  return true;
}

template <int KS1, int KS2, bool W4>
static int run_stream_layer(const GemmArgs& g1, const GemmArgs& g2, LayerSync ls, hipStream_t stream) {
  int cap1, cap2;
  size_t sh1, sh2;
  const size_t r1 = cu_ring_bytes<KS1, W4>(), r2 = cu_ring_bytes<KS2, W4>();
  ls.lists_at = (int)(r1 > r2 ? r1 : r2);
  if (!cu_window<KS1, W4>(g1, ls.lists_at, &cap1, &sh1) || !cu_window<KS2, W4>(g2, ls.lists_at, &cap2, &sh2)) {
    set_last_error("stream_layer: the windows do not fit in LDS");
    return kUnsupported;
  }
  const size_t shmem = sh1 > sh2 ? sh1 : sh2;
  auto kern = stream_layer_kernel<KS1, KS2, W4>;
  const int st = ensure_dynamic_lds((const void*)kern, shmem, "stream_layer");
  if (st != kOk) return st;
  const int cus = device_cu_count();
  if (cus <= 0) return kLaunchError;
  if (cus > kMaxLayerRanges) {
    set_last_error("stream_layer: %d CUs, more than the %d claim words of the sync area", cus, kMaxLayerRanges);
    return kUnsupported;
  }
  kern<<<dim3(cus), dim3(W4 ? kCuThreadsW4 : kCuThreads), shmem, stream>>>(g1, g2, cap1, cap2, ls);
  return launch_status("stream_layer");
}

// (H, I): the Qwen3-Omni thinker (2048, 768) and talker (1024, 384) MoE
// shapes; int4 weights need I % 256 == 0.
bool stream_layer_supported(int64_t H, int64_t I, int64_t slots, int E, bool int4) {
  const bool shape = (H == 2048 && I == 768) || (!int4 && H == 1024 && I == 384);
  return shape && slots <= kStreamMaxIdsSlots && E <= 1024;
}

int launch_stream_layer(const GemmArgs& g1, const GemmArgs& g2, bool int4, int* sync_words, hipStream_t stream) {
  const bool rows_ok = int4 ? (!g1.a_q16 && !g1.a_scale) : (g1.a_q16 && g1.a_scale);
  if (!stream_layer_supported(g1.K, g1.inter, g1.M, g1.num_experts, int4) || !g1.topk_ids || !g2.topk_ids ||
      !rows_ok || g2.a_scale || g2.K != g1.inter || g2.N != g1.K || !sync_words) {
    set_last_error("stream_layer: unsupported configuration");
    return kUnsupported;
  }
  LayerSync ls;
  ls.done = sync_words;
  ls.err = sync_words + g1.num_experts;
  ls.claim = sync_words + layer_claim_base(g1.num_experts);
  ls.gate_ipe = g1.inter / 8;
  ls.down_ipe = g2.N / 16;
  ls.mode = g_layer_test_mode.load(std::memory_order_relaxed);
  if (int4) return run_stream_layer<16, 6, true>(g1, g2, ls, stream);
  return g1.K == 2048 ? run_stream_layer<16, 6, false>(g1, g2, ls, stream)
                      : run_stream_layer<8, 3, false>(g1, g2, ls, stream);
}

int layer_wait_failures(int* count) {
  if (!count) {
    set_last_error("moe_layer_wait_failures: null pointer");
    return kInvalidArgument;
  }
  if (hipMemcpyFromSymbol(count, HIP_SYMBOL(g_layer_wait_failures), sizeof(int), 0, hipMemcpyDeviceToHost) !=
      hipSuccess) {
    set_last_error("moe_layer_wait_failures: reading the counter failed");
    return kLaunchError;
  }
  return kOk;
}

int launch_stream_int4_cu(const GemmArgs& a, int epi, hipStream_t stream) {
  if (!a.topk_ids || a.M > kStreamMaxIdsSlots || a.num_experts > 1024 || a.K % 256 != 0 ||
      (epi == EPI_ACT ? a.inter % 8 != 0 : a.N % 16 != 0)) {
    set_last_error("stream_int4: needs router ids, at most %lld slots, K %% 256 == 0",
                   (long long)kStreamMaxIdsSlots);
    return kUnsupported;
  }
  int st = kOk;
  bool done = false;
  switch (a.K / 128) {
    case 2: done = try_stream_fp8_cu<2>(a, epi, stream, &st, true); break;
    case 4: done = try_stream_fp8_cu<4>(a, epi, stream, &st, true); break;
    case 6: done = try_stream_fp8_cu<6>(a, epi, stream, &st, true); break;
    case 8: done = try_stream_fp8_cu<8>(a, epi, stream, &st, true); break;
    case 12: done = try_stream_fp8_cu<12>(a, epi, stream, &st, true); break;
    case 16: done = try_stream_fp8_cu<16>(a, epi, stream, &st, true); break;
  }
  if (!done) {
    set_last_error("stream_int4: unsupported shape (K=%d)", a.K);
    return kUnsupported;
  }
  return st;
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
    if (!exact)                                                                             \
      return epi == EPI_ACT ? run_stream_fp8<EPI_ACT, KS, false, false>(a, stream)          \
                            : run_stream_fp8<EPI_STORE, KS, false, false>(a, stream);       \
    if (aq)                                                                                 \
      return epi == EPI_ACT ? run_stream_fp8<EPI_ACT, KS, true, true>(a, stream)            \
                            : run_stream_fp8<EPI_STORE, KS, true, true>(a, stream);         \
    return epi == EPI_ACT ? run_stream_fp8<EPI_ACT, KS, true, false>(a, stream)             \
                          : run_stream_fp8<EPI_STORE, KS, true, false>(a, stream);
  // A with a_scale: e4m3fn rows already quantised per group of 128;
  // otherwise bf16 rows, quantised while they are staged.
  const bool aq = a.a_scale != nullptr;
  if (aq && !exact) {
    set_last_error("stream_fp8: pre-quantised activations need the exact path");
    return kUnsupported;
  }
  if (exact && a.topk_ids && a.M <= kStreamMaxIdsSlots) {
    int st = kOk;
    bool done = false;
    switch (a.K / 128) {
      case 1: done = try_stream_fp8_cu<1>(a, epi, stream, &st); break;
      case 2: done = try_stream_fp8_cu<2>(a, epi, stream, &st); break;
      case 3: done = try_stream_fp8_cu<3>(a, epi, stream, &st); break;
      case 4: done = try_stream_fp8_cu<4>(a, epi, stream, &st); break;
      case 6: done = try_stream_fp8_cu<6>(a, epi, stream, &st); break;
      case 8: done = try_stream_fp8_cu<8>(a, epi, stream, &st); break;
      case 12: done = try_stream_fp8_cu<12>(a, epi, stream, &st); break;
      case 16: done = try_stream_fp8_cu<16>(a, epi, stream, &st); break;
    }
    if (done) return st;
  }
  if (a.a_q16) {
    set_last_error("stream_fp8: widened activations need the CU-resident kernel (exact, router ids, "
                   "at most %lld slots)", (long long)kStreamMaxIdsSlots);
    return kUnsupported;
  }
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

#ifdef MSTAR_TIMELINE
extern "C" int mstar_debug_timeline(uint64_t* dst, size_t n) {
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(mstar::g_timeline), n * 8, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 1;
}
#endif
