// Large-tile FP8 GEMM for prefill-sized MoE layers and the dense W8A8 GEMM.
//
// One 512-thread workgroup (8 waves, 4 x 2) owns a 256 (tokens) x 128
// (weight rows) output tile and walks K in 128-wide steps -- exactly one FP8
// scale block per step.
//
// Data movement.  A step's operands (32 KB of activations, 16 KB of weights
// and, when block-scaled, the step's activation and weight scales) go
// straight from global memory into LDS with gfx950's LDS-DMA loads
// (global_load_lds_dwordx4: lane l's bytes land at base + 16 l), into a ring
// of three stages: while step k computes, steps k+1 and k+2 are in flight and
// no VGPRs or LDS-store instructions are spent on staging.  Rows are 128
// bytes with the 16-byte chunks XOR-swizzled by (row & 7), so the lanes of a
// ds_read_b128 phase hit distinct banks.  One barrier per step.
//
// Math.  Each wave owns a 64 x 64 sub-tile as 2 x 2 tiles of 32 x 32, two
// chained v_mfma_f32_32x32x64_f8f6f4 per tile per step.  The product is
// computed transposed (weights as the MFMA's A operand, tokens as B) so that
// each lane holds one token column: with block-scaled operands (MoE) a
// step's partial is promoted with one factor s_a[token, kb] * s_w[block, kb]
// per lane -- 16 FMAs per tile per step, which overlap the MFMA pipe.
// Per-token x per-channel operands (dense): the MFMAs chain into the
// accumulator and the scales are applied in the epilogue.
//
// Epilogue.  Each wave converts its 64 x 64 block to bf16 in LDS, then every
// lane stores 16 contiguous bytes of an output row.
//
// Grouped mode follows the reference's fused_moe_kernel contract
// (mstar/utils/fused_moe/kernels.py:83-138): one 256-row block of
// `sorted_ids` per tile row, A row = slot / top_k, padding masked, blocks past
// num_tokens_post_padded exit at once.
#include "common.h"
#include "launch.h"

namespace mstar {

constexpr int kBigBM = 256, kBigBN = 128;
constexpr int kBigWM = 4, kBigWN = 2;  // wave grid; wave tile 64 x 64
constexpr int kBigStages = 3;
// Stage: A tile, B tile (128-byte rows), A-row scales [256], weight-block
// scales [64] (4 used: one per (wave column, 32-row tile)).
constexpr int kBigAsOff = (kBigBM + kBigBN) * 128;
constexpr int kBigBsOff = kBigAsOff + kBigBM * 4;
constexpr int kBigStageBytes = kBigBsOff + 64 * 4;
constexpr size_t kBigLds = (size_t)kBigStages * kBigStageBytes + 2 * kBigBM * sizeof(int);

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// Workgroup id -> tile id such that XCD x (= id % 8) walks tiles
// [x * G/8, (x+1) * G/8) in order (the remainder goes to the last ids).
__device__ inline int xcd_remap(int id, int grid) {
  constexpr int kXcd = 8;
  const int per = grid / kXcd;
  if (id >= per * kXcd) return id;
  return (id % kXcd) * per + id / kXcd;
}

// 32 bytes: logical 16-byte chunks c and c+1 of swizzled LDS row `row`.
__device__ __forceinline__ v8i lds_frag_swz(const uint8_t* row_base, int row, int c) {
  const int sw = row & 7;
  const v4i lo = *(const v4i*)(row_base + ((c ^ sw) << 4));
  const v4i hi = *(const v4i*)(row_base + (((c + 1) ^ sw) << 4));
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <int EPI, bool GROUPED, bool BLOCKSCALE>
__global__ __launch_bounds__(512) void gemm_fp8_big_kernel(GemmArgs p) {
  constexpr int BM = kBigBM, BN = kBigBN, WN = kBigWN, WTM = BM / kBigWM, WTN = BN / kBigWN;
  constexpr int MB = WTM / 32, NB = WTN / 32;      // 32x32 MFMA tiles per wave
  constexpr int AI = BM / 8 / 8, BI = BN / 8 / 8;  // 1 KB DMA instructions per wave per step
  static_assert(EPI != EPI_ACT || NB == 2, "fused activation pairs one gate and one up tile");
  static_assert(WN * NB <= 64, "weight-scale slots");
  extern __shared__ __align__(16) uint8_t smem[];
  int* sRow = (int*)(smem + (size_t)kBigStages * kBigStageBytes);
  int* sSlot = sRow + BM;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, lh = lane >> 5;

  const int n_tiles = EPI == EPI_ACT ? (p.inter + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
  // Workgroups are dealt round-robin to the 8 XCDs; give each XCD one
  // contiguous run of tiles so the n-tiles of an m-block (which share A rows)
  // and neighbouring m-blocks of an expert (which share weights) meet in the
  // same L2.
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int nt = tile % n_tiles;
  const int mb = tile / n_tiles;
  int expert = 0;
  if constexpr (GROUPED) {
    if ((int64_t)mb * BM >= (int64_t)(*p.ntpp)) return;
    expert = p.expert_ids[mb];
  } else {
    if ((int64_t)mb * BM >= p.M) return;
  }
  for (int r = tid; r < BM; r += 512) {
    int arow = -1, slot = -1;
    if constexpr (GROUPED) {
      const int s = p.sorted_ids[(int64_t)mb * BM + r];
      if (s < p.M) { slot = s; arow = s / p.top_k; }
    } else {
      const int64_t m = (int64_t)mb * BM + r;
      if (m < p.M) { slot = (int)m; arow = (int)m; }
    }
    sRow[r] = arow;
    sSlot[r] = slot;
  }
  __syncthreads();

  // Weight row of B-tile row rho; -1 past the edge.  With the fused
  // activation each wave column's 64 rows are 32 gate rows then the matching
  // 32 up rows.
  auto brow_of = [&](int rho) -> int {
    if constexpr (EPI == EPI_ACT) {
      const int ww = rho / WTN, q = rho % WTN;
      const int gcol = nt * (BN / 2) + ww * (WTN / 2) + (q % (WTN / 2));
      if (gcol >= p.inter) return -1;
      return q < WTN / 2 ? gcol : p.inter + gcol;
    } else {
      const int n = nt * BN + rho;
      return n < p.N ? n : -1;
    }
  };

  // DMA instruction q of this wave fills tile rows [R, R + 8), R = wave*rows +
  // 8 q: lane l's 16 bytes land at row R + l/8, physical chunk l%8, which
  // holds logical chunk (l%8) ^ (l/8) (= (l%8) ^ (row & 7)).  Padding rows
  // read row 0: their outputs are never stored, and branch-free loads keep
  // the wait counts exact.
  const uint32_t lchunk = (uint32_t)(((lane & 7) ^ (lane >> 3)) * 16);
  const uint8_t* a_base = (const uint8_t*)p.A;
  const uint8_t* b_base = (const uint8_t*)p.B + (int64_t)expert * p.b_estride;
  uint32_t a_off[AI], b_off[BI];
#pragma unroll
  for (int q = 0; q < AI; ++q) {
    const int ar = sRow[wave * (BM / 8) + q * 8 + (lane >> 3)];
    a_off[q] = (uint32_t)((int64_t)(ar >= 0 ? ar : 0) * p.lda) + lchunk;
  }
#pragma unroll
  for (int q = 0; q < BI; ++q) {
    const int br = brow_of(wave * (BN / 8) + q * 8 + (lane >> 3));
    b_off[q] = (uint32_t)((int64_t)(br >= 0 ? br : 0) * p.ldb) + lchunk;
  }
  // Scales ride the same DMA stream (a plain global load here would make
  // the compiler drain every outstanding DMA before using it).  Waves 0-3
  // move the 256 A-row scales, wave 4 the weight-block scales: lane l the
  // block of (wave column (l/2)%WN, tile l%2).
  const float* sc_src = nullptr;
  if constexpr (BLOCKSCALE) {
    if (wave < 4) {
      const int ar = sRow[wave * 64 + lane];
      sc_src = p.a_scale + (int64_t)(ar >= 0 ? ar : 0) * p.ld_as;
    } else {
      const int ww = (lane >> 1) % WN, j = lane & 1;
      const int r = brow_of(ww * WTN + j * 32);
      sc_src = (const float*)p.b_scale + (int64_t)expert * p.bs_estride +
               (int64_t)(r < 0 ? 0 : r / 128) * p.bs_ld;
    }
  }
  constexpr int kScaleWaves = 5;

  auto issue = [&](int kb) {
    uint8_t* st = smem + (kb % kBigStages) * kBigStageBytes;
#pragma unroll
    for (int q = 0; q < AI; ++q)
      __builtin_amdgcn_global_load_lds((const void*)(a_base + a_off[q] + kb * 128),
                                       (lds_void_ptr)(st + (wave * (BM / 8) + q * 8) * 128), 16, 0, 0);
#pragma unroll
    for (int q = 0; q < BI; ++q)
      __builtin_amdgcn_global_load_lds((const void*)(b_base + b_off[q] + kb * 128),
                                       (lds_void_ptr)(st + BM * 128 + (wave * (BN / 8) + q * 8) * 128),
                                       16, 0, 0);
    if constexpr (BLOCKSCALE) {
      if (wave < 4)
        __builtin_amdgcn_global_load_lds((const void*)(sc_src + kb),
                                         (lds_void_ptr)(st + kBigAsOff + wave * 256), 4, 0, 0);
      else if (wave == 4)
        __builtin_amdgcn_global_load_lds((const void*)(sc_src + kb), (lds_void_ptr)(st + kBigBsOff),
                                         4, 0, 0);
    }
  };
  // Wait until this wave's DMA of the oldest outstanding step has landed; if
  // `next` the following step's stays in flight.
  constexpr int kPer = AI + BI;
  auto wait_step = [&](bool next) {
    if (!next) {
      wait_vmcnt<0>();
    } else if (BLOCKSCALE && wave < kScaleWaves) {
      wait_vmcnt<kPer + 1>();
    } else {
      wait_vmcnt<kPer>();
    }
  };

  // acc[i][j]: the transposed 32x32 tile (weight rows x token columns).
  v16f acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = v16f{};

  // Block-scaled promotion is software-pipelined so that the matrix pipe
  // never waits on the VALU: the partials of row tile i are promoted while
  // the MFMAs of row tile i+1 run, and the last row tile's partials (tp,
  // with factors fp) are promoted during the first MFMAs of the next step.
  v16f tp[NB];
  float fp[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) { tp[j] = v16f{}; fp[j] = 0.f; }
  // Promotion of eight accumulator registers of tile j of row tile i.
  auto promote8 = [&](int i, int j, int half) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      acc[i][j][half * 8 + e] = __builtin_fmaf(tp[j][half * 8 + e], fp[j], acc[i][j][half * 8 + e]);
  };
  // Pins the instruction order written in the source: each MFMA is followed
  // by the slice of VALU promotion that runs in its shadow.
  auto fence_sched = [] { __builtin_amdgcn_sched_barrier(0); };

  const int KB = p.K / 128;
  issue(0);
  if (KB > 1) issue(1);
  for (int kb = 0; kb < KB; ++kb) {
    wait_step(kb + 1 < KB);
    // Step kb has landed for every wave, and every wave is past step kb-1,
    // whose stage the next issue overwrites.  A bare s_barrier: the
    // workgroup fence of __syncthreads() would drain the DMA still in flight.
    lds_barrier();
    if (kb + 2 < KB) issue(kb + 2);
    const uint8_t* st = smem + (kb % kBigStages) * kBigStageBytes;
    const uint8_t* sA = st;
    const uint8_t* sB = st + BM * 128;
    v8i wf[NB][2];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int r = wn * WTN + j * 32 + l32;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) wf[j][kh] = lds_frag_swz(sB + r * 128, r, kh * 4 + lh * 2);
    }
    if constexpr (BLOCKSCALE) {
      static_assert(NB == 2, "promotion schedule assumes two weight tiles per wave");
      float sw[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j) sw[j] = ((const float*)(st + kBigBsOff))[wn * 2 + j];
      v8i x[2][2];
      float sa[2];
      auto load_x = [&](int i) {
        const int r = wm * WTM + i * 32 + l32;
        x[i & 1][0] = lds_frag_swz(sA + r * 128, r, lh * 2);
        x[i & 1][1] = lds_frag_swz(sA + r * 128, r, 4 + lh * 2);
        sa[i & 1] = ((const float*)(st + kBigAsOff))[r];  // this lane's token
      };
      load_x(0);
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        // The previous row tile: of this step, or the last of the previous step.
        const int ip = i == 0 ? MB - 1 : i - 1;
        const v8i* xi = x[i & 1];
        v16f t[NB];
        fence_sched();
        t[0] = mfma_fp8_32x32x64(wf[0][0], xi[0], v16f{});
        if (i + 1 < MB) load_x(i + 1);
        promote8(ip, 0, 0);
        fence_sched();
        t[1] = mfma_fp8_32x32x64(wf[1][0], xi[0], v16f{});
        promote8(ip, 0, 1);
        fence_sched();
        t[0] = mfma_fp8_32x32x64(wf[0][1], xi[1], t[0]);
        promote8(ip, 1, 0);
        fence_sched();
        t[1] = mfma_fp8_32x32x64(wf[1][1], xi[1], t[1]);
        promote8(ip, 1, 1);
        fence_sched();
#pragma unroll
        for (int j = 0; j < NB; ++j) { tp[j] = t[j]; fp[j] = sa[i & 1] * sw[j]; }
      }
    } else {
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const int r = wm * WTM + i * 32 + l32;
        const v8i x0 = lds_frag_swz(sA + r * 128, r, lh * 2);
        const v8i x1 = lds_frag_swz(sA + r * 128, r, 4 + lh * 2);
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = mfma_fp8_32x32x64(wf[j][0], x0, acc[i][j]);
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = mfma_fp8_32x32x64(wf[j][1], x1, acc[i][j]);
      }
    }
  }
  if constexpr (BLOCKSCALE) {
#pragma unroll
    for (int j = 0; j < NB; ++j) { promote8(MB - 1, j, 0); promote8(MB - 1, j, 1); }
  }
  __syncthreads();  // every wave is done with the ring: reuse it below

  // ---------------------------------------------------------------- epilogue
  // Lane (l32, lh), register e of tile (i, j): token row wm*WTM + i*32 + l32,
  // weight column wn*WTN + j*32 + 8*(e/4) + 4*lh + (e%4).  The wave writes
  // its bf16 block [64 tokens][OW columns] to a private LDS area (rows padded
  // by 16 bytes), then each lane stores 16 contiguous bytes of one row.
  constexpr int OW = EPI == EPI_ACT ? WTN / 2 : WTN;  // output columns per wave
  constexpr int OWB = OW * 2;                         // bytes per output row
  constexpr int OLD = OWB + 16;                       // LDS row pitch
  uint8_t* so = smem + wave * (WTM * OLD);
  float rscale[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const int slot = sSlot[wm * WTM + i * 32 + l32];
    if constexpr (EPI == EPI_DENSE) rscale[i] = slot >= 0 ? p.a_scale[slot] : 0.f;
    else if constexpr (EPI == EPI_STORE)
      rscale[i] = (p.mul_routed && slot >= 0) ? load_weight_any(p.topk_w, p.topk_w_dtype, slot) : 1.f;
    else rscale[i] = 1.f;
  }
  float csc[NB][4][4];  // dense: per-channel weight scales of this lane's columns
  if constexpr (EPI == EPI_DENSE) {
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int gc = nt * BN + wn * WTN + j * 32 + 8 * q + 4 * lh + e;
          csc[j][q][e] = gc < p.N ? ((const float*)p.b_scale)[gc] : 0.f;
        }
  }
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    uint8_t* orow = so + (i * 32 + l32) * OLD;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if constexpr (EPI == EPI_ACT) {
        uint32_t w2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint32_t two = 0;
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int r = 4 * q + 2 * h + e;
            const float g = round_bf16(acc[i][0][r]);
            const float u = round_bf16(acc[i][1][r]);
            const float a = round_bf16(p.activation == 0 ? act_f32<0>(g) : act_f32<1>(g));
            two |= (uint32_t)f32_to_bf16_bits(a * u) << (16 * e);
          }
          w2[h] = two;
        }
        *(uint2*)(orow + (8 * q + 4 * lh) * 2) = make_uint2(w2[0], w2[1]);
      } else {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int col = j * 32 + 8 * q + 4 * lh;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = acc[i][j][4 * q + e] * rscale[i];
            if constexpr (EPI == EPI_DENSE) v[e] *= csc[j][q][e];
          }
          const uint32_t lo = (uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
          const uint32_t hi = (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16);
          *(uint2*)(orow + col * 2) = make_uint2(lo, hi);
        }
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint16_t* C = (uint16_t*)p.C;
  const int col0 = EPI == EPI_ACT ? nt * (BN / 2) + wn * (WTN / 2) : nt * BN + wn * WTN;
  const int ncols = EPI == EPI_ACT ? p.inter : p.N;
  constexpr int CPR = OWB / 16;  // 16-byte chunks per output row
  const bool vec_ok = (p.ldc & 7) == 0;
#pragma unroll
  for (int it = 0; it < WTM * CPR / 64; ++it) {
    const int c = it * 64 + lane;
    const int row = c / CPR, ch = c % CPR;
    const int slot = sSlot[wm * WTM + row];
    const int gc = col0 + ch * 8;
    if (slot < 0 || gc >= ncols) continue;
    const v4i v = *(const v4i*)(so + row * OLD + ch * 16);
    uint16_t* dst = C + (int64_t)slot * p.ldc + gc;
    if (gc + 8 <= ncols && vec_ok) {
      *(v4i*)dst = v;
    } else {
      const uint16_t* e = (const uint16_t*)&v;
      for (int k = 0; k < 8 && gc + k < ncols; ++k) dst[k] = e[k];
    }
  }
}

template <int EPI, bool GROUPED, bool BLOCKSCALE>
static int run_big(const GemmArgs& a, hipStream_t stream) {
  auto kern = gemm_fp8_big_kernel<EPI, GROUPED, BLOCKSCALE>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)kBigLds) != hipSuccess) {
      set_last_error("gemm_fp8_big: cannot reserve %zu bytes of LDS", kBigLds);
      return kLaunchError;
    }
    attr_set = true;
  }
  const int n_tiles = EPI == EPI_ACT ? (a.inter + kBigBN / 2 - 1) / (kBigBN / 2) : (a.N + kBigBN - 1) / kBigBN;
  const int64_t m_blocks = GROUPED ? a.m_blocks : (a.M + kBigBM - 1) / kBigBM;
  if (m_blocks == 0) return kOk;
  const int64_t grid = m_blocks * n_tiles;
  if (grid >= ((int64_t)1 << 31)) {
    set_last_error("gemm_fp8_big: grid too large");
    return kUnsupported;
  }
  kern<<<dim3((unsigned)grid), dim3(512), kBigLds, stream>>>(a);
  return launch_status("gemm_fp8_big");
}

int launch_gemm_fp8_big(const GemmArgs& a, int epi, bool grouped, hipStream_t stream) {
  if (a.K <= 0 || a.K % 128 != 0 || (epi == EPI_ACT && (a.N != 2 * a.inter))) {
    set_last_error("gemm_fp8_big: K must be a positive multiple of 128 (and N == 2 * inter)");
    return kInvalidArgument;
  }
  // Row offsets are 32-bit byte offsets.
  const int64_t a_rows = grouped ? (a.M + a.top_k - 1) / (a.top_k > 0 ? a.top_k : 1) : a.M;
  if (a_rows * a.lda >= ((int64_t)1 << 32) || (int64_t)a.N * a.ldb >= ((int64_t)1 << 32)) {
    set_last_error("gemm_fp8_big: operand larger than 4 GiB");
    return kUnsupported;
  }
  if (grouped) {
    if (epi == EPI_ACT) return run_big<EPI_ACT, true, true>(a, stream);
    if (epi == EPI_STORE) return run_big<EPI_STORE, true, true>(a, stream);
  } else if (epi == EPI_DENSE) {
    return run_big<EPI_DENSE, false, false>(a, stream);
  }
  set_last_error("gemm_fp8_big: unsupported epilogue %d (grouped=%d)", epi, (int)grouped);
  return kUnsupported;
}

}  // namespace mstar
