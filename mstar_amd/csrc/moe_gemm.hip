// Grouped (MoE) and dense GEMMs on CDNA4 MFMA.
//
// Two kernels share one argument block (GemmArgs, launch.h):
//
// tile_gemm_kernel -- LDS-tiled MFMA GEMM for large token counts.  A
//   workgroup (4 waves) owns a BM x BN output tile; K advances 128 elements
//   per step, which is exactly one FP8 scale block, so the per-block dequant
//   scale s_a[row] * s_w[nblock] is applied to each 16x16x128 partial
//   product as it is produced.  In grouped mode the BM rows are one
//   expert-aligned block of `sorted_ids` (the moe_align_block_size output),
//   mirroring fused_moe_kernel (mstar/utils/fused_moe/kernels.py:36-138):
//   A row = slot / top_k, padding slots (>= numel) are masked, and blocks at
//   or past num_tokens_post_padded exit at once (kernels.py:93-96).
//   Epilogues: plain store (optionally times the routed weight,
//   kernels.py:129-133), fused activation-and-mul (the act_and_mul_kernel of
//   kernels.py:244-276 applied to the tile; the tile holds matching gate and
//   up columns), and the dense per-token x per-channel FP8 scaling.
//
// stream_gemm_kernel -- weight streaming for decode-sized batches.  One
//   workgroup per (n-tile, expert); each wave keeps its 16 weight rows for
//   the whole K in registers (issued up front, so a CU has hundreds of KB
//   in flight), the expert's token rows are staged (and, for FP8, quantised
//   per 128-group) in LDS, and every weight byte is read from HBM once no
//   matter how many tokens chose the expert.
#include "common.h"
#include "launch.h"

#include <type_traits>

namespace mstar {

// ---------------------------------------------------------------------------
// Shared helpers
// ---------------------------------------------------------------------------
__device__ inline float load_weight(const void* w, int dtype, int64_t i) {
  return load_weight_any(w, dtype, i);
}

// 32 bytes from a 16-byte aligned address (LDS rows are padded to 16 bytes,
// not 32, so a plain v8i dereference would claim too much alignment).
__device__ inline v8i load_v8i_a16(const uint8_t* p) {
  v4i lo = *(const v4i*)p, hi = *(const v4i*)(p + 16);
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// 8 int4 nibbles (u = q + 8) -> 8 16-bit values bf16/fp16(q * s).
template <int DT>
__device__ inline v8s dequant_int4x8(uint32_t word, float s) {
  if constexpr (DT == kBF16) return int4x8_dequant_bf16(word, s, -8.f * s);
  v8s r;
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    float q = (float)((int)((word >> (4 * n)) & 0xfu) - 8);
    r[n] = (short)f32_to_h16<DT>(q * s);
  }
  return r;
}

template <int AK, int BK>
struct Engine {
  static constexpr bool kFp8 = AK != A_H16;
  static constexpr int kRowBytes = kFp8 ? 128 : 256;  // bytes per row per 128-K step
  static constexpr int kLdr = kRowBytes + 16;         // padded LDS row stride
};

template <int BM>
struct WaveGrid {
  static constexpr int WM = BM >= 32 ? 2 : 1;
  static constexpr int WN = 4 / WM;
};

// ---------------------------------------------------------------------------
// Tiled GEMM
// ---------------------------------------------------------------------------
template <int AK, int BK, int EPI, int DT, bool GROUPED, int BM, int BN>
__global__ __launch_bounds__(256) void tile_gemm_kernel(GemmArgs p) {
  using En = Engine<AK, BK>;
  constexpr bool FP8 = En::kFp8;
  constexpr int RB = En::kRowBytes, LDR = En::kLdr;
  constexpr int WM = WaveGrid<BM>::WM, WN = WaveGrid<BM>::WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int MS = WTM / 16, NS = WTN / 16;
  constexpr int ES = FP8 ? 1 : 2;                 // A/B element bytes in LDS
  constexpr int CPR = RB / 16;                    // 16-byte chunks per LDS row
  constexpr int CA = BM * CPR / 256;              // A chunks per thread
  constexpr int BG_CPR = (BK == B_INT4G) ? 4 : CPR;  // global chunks per B row
  constexpr int CB = BN * BG_CPR / 256;           // B chunks per thread
  static_assert(CA >= 1 && CB >= 1, "tile too small for 256 threads");
  static_assert(EPI != EPI_ACT || NS % 2 == 0, "act epilogue needs gate/up subtile pairs");

  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* sA = smem;
  uint8_t* sB = sA + BM * LDR;
  float* sAs = (float*)(sB + BN * LDR);
  int* sRow = (int*)(sAs + BM);
  int* sSlot = sRow + BM;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int l16 = lane & 15, lg = lane >> 4;

  const int n_tiles = (EPI == EPI_ACT) ? (p.inter + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
  const int nt = blockIdx.x % n_tiles;
  const int mb = blockIdx.x / n_tiles;
  int expert = 0;
  if constexpr (GROUPED) {
    if ((int64_t)mb * BM >= (int64_t)(*p.ntpp)) return;
    expert = p.expert_ids[mb];
  } else {
    if ((int64_t)mb * BM >= p.M) return;
  }

  for (int r = tid; r < BM; r += 256) {
    int arow = -1, slot = -1;
    if constexpr (GROUPED) {
      int s = p.sorted_ids[(int64_t)mb * BM + r];
      if (s < p.M) { slot = s; arow = s / p.top_k; }
    } else {
      int64_t m = (int64_t)mb * BM + r;
      if (m < p.M) { slot = (int)m; arow = (int)m; }
    }
    sRow[r] = arow;
    sSlot[r] = slot;
  }
  __syncthreads();

  // Weight row of LDS B-tile row rho (-1 when out of range).
  auto brow_of = [&](int rho) -> int {
    if constexpr (EPI == EPI_ACT) {
      const int half = WTN / 2;
      const int ww = rho / WTN, q = rho % WTN;
      const int gcol = nt * (BN / 2) + ww * half + (q % half);
      if (gcol >= p.inter) return -1;
      return q < half ? gcol : p.inter + gcol;
    } else {
      const int n = nt * BN + rho;
      return n < p.N ? n : -1;
    }
  };

  const uint8_t* Ab = (const uint8_t*)p.A;
  const int64_t a_rowbytes = p.lda * ES;
  int a_row[CA], a_col[CA];
  const uint8_t* a_ptr[CA];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    int c = tid + i * 256;
    a_row[i] = c / CPR;
    a_col[i] = c % CPR;
    int src = sRow[a_row[i]];
    a_ptr[i] = src >= 0 ? Ab + (int64_t)src * a_rowbytes + a_col[i] * 16 : nullptr;
  }
  int b_row[CB], b_col[CB];
  const uint8_t* b_ptr[CB];
  const uint16_t* bs16_ptr[CB];
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    int c = tid + i * 256;
    b_row[i] = c / BG_CPR;
    b_col[i] = c % BG_CPR;
    int br = brow_of(b_row[i]);
    bs16_ptr[i] = nullptr;
    if (br < 0) {
      b_ptr[i] = nullptr;
    } else if constexpr (BK == B_INT4G) {
      b_ptr[i] = (const uint8_t*)((const int32_t*)p.B + (int64_t)expert * p.b_estride +
                                  (int64_t)br * p.ldb) + b_col[i] * 16;
      bs16_ptr[i] = (const uint16_t*)p.b_scale + (int64_t)expert * p.bs_estride +
                    (int64_t)br * p.bs_ld;
    } else {
      b_ptr[i] = (const uint8_t*)p.B + ((int64_t)expert * p.b_estride + (int64_t)br * p.ldb) * ES +
                 b_col[i] * 16;
    }
  }
  // FP8 block scales: one row pointer per wave n-subtile.
  const float* sw_ptr[NS];
  if constexpr (BK == B_FP8BLK) {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      int br = brow_of(wn * WTN + j * 16);
      sw_ptr[j] = (const float*)p.b_scale + (int64_t)expert * p.bs_estride +
                  (int64_t)(br < 0 ? 0 : br / 128) * p.bs_ld;
    }
  }
  const float* as_ptr = nullptr;
  if constexpr (AK == A_FP8G) {
    if (tid < BM && sRow[tid] >= 0) as_ptr = p.a_scale + (int64_t)sRow[tid] * p.ld_as;
  }

  // 16-bit operands take any K: the last 128-K step (and every step when a
  // row is not 16-byte aligned) loads element by element and zero-fills the
  // columns at or past K, so both operands contribute exact zeros there.
  constexpr bool KTAIL = AK == A_H16 && BK == B_H16;
  bool vec_ok = true;
  if constexpr (KTAIL)
    vec_ok = ((p.lda | p.ldb | p.b_estride) & 7) == 0 && (((uintptr_t)p.A | (uintptr_t)p.B) & 15) == 0;
  auto load_h16_chunk = [&](const uint8_t* ptr, int col, int kb) -> v4i {
    v4i r = {0, 0, 0, 0};
    if (!ptr) return r;
    const uint16_t* e = (const uint16_t*)(ptr + (int64_t)kb * RB);
    const int k0 = kb * 128 + col * 8;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const uint32_t lo = k0 + 2 * n < p.K ? e[2 * n] : 0u;
      const uint32_t hi = k0 + 2 * n + 1 < p.K ? e[2 * n + 1] : 0u;
      r[n] = (int)(lo | (hi << 16));
    }
    return r;
  };

  v4i ra[CA], rb[CB];
  float ras = 0.f;
  float rbs[CB];
  auto load_step = [&](int kb) {
    if constexpr (KTAIL) {
      if (!vec_ok || (kb + 1) * 128 > p.K) {
#pragma unroll
        for (int i = 0; i < CA; ++i) ra[i] = load_h16_chunk(a_ptr[i], a_col[i], kb);
#pragma unroll
        for (int i = 0; i < CB; ++i) rb[i] = load_h16_chunk(b_ptr[i], b_col[i], kb);
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < CA; ++i)
      ra[i] = a_ptr[i] ? *(const v4i*)(a_ptr[i] + (int64_t)kb * RB) : v4i{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      if constexpr (BK == B_INT4G) {
        rb[i] = b_ptr[i] ? *(const v4i*)(b_ptr[i] + (int64_t)kb * 64) : v4i{0, 0, 0, 0};
        rbs[i] = bs16_ptr[i] ? h16_to_f32<DT>(bs16_ptr[i][kb]) : 0.f;
      } else {
        rb[i] = b_ptr[i] ? *(const v4i*)(b_ptr[i] + (int64_t)kb * RB) : v4i{0, 0, 0, 0};
      }
    }
    if constexpr (AK == A_FP8G) ras = as_ptr ? as_ptr[kb] : 0.f;
  };
  auto store_step = [&]() {
#pragma unroll
    for (int i = 0; i < CA; ++i) *(v4i*)(sA + a_row[i] * LDR + a_col[i] * 16) = ra[i];
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      if constexpr (BK == B_INT4G) {
        uint8_t* dst = sB + b_row[i] * LDR + b_col[i] * 64;
#pragma unroll
        for (int w = 0; w < 4; ++w) *(v8s*)(dst + w * 16) = dequant_int4x8<DT>((uint32_t)rb[i][w], rbs[i]);
      } else {
        *(v4i*)(sB + b_row[i] * LDR + b_col[i] * 16) = rb[i];
      }
    }
    if constexpr (AK == A_FP8G) {
      if (tid < BM) sAs[tid] = ras;
    }
  };

  v4f acc[MS][NS];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NS; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int KB = KTAIL ? (p.K + 127) / 128 : p.K / 128;
  load_step(0);
  for (int kb = 0; kb < KB; ++kb) {
    store_step();
    __syncthreads();
    if (kb + 1 < KB) load_step(kb + 1);
    if constexpr (FP8) {
      v8i af[MS], bf[NS];
#pragma unroll
      for (int i = 0; i < MS; ++i)
        af[i] = load_v8i_a16(sA + (wm * WTM + i * 16 + l16) * LDR + lg * 32);
#pragma unroll
      for (int j = 0; j < NS; ++j)
        bf[j] = load_v8i_a16(sB + (wn * WTN + j * 16 + l16) * LDR + lg * 32);
      if constexpr (AK == A_FP8G) {
        float sw[NS];
#pragma unroll
        for (int j = 0; j < NS; ++j) sw[j] = sw_ptr[j][kb];
#pragma unroll
        for (int i = 0; i < MS; ++i) {
          v4f sa = *(const v4f*)(sAs + wm * WTM + i * 16 + lg * 4);
#pragma unroll
          for (int j = 0; j < NS; ++j) {
            v4f t = mfma_fp8_16x16x128(af[i], bf[j], v4f{0.f, 0.f, 0.f, 0.f});
            acc[i][j] += t * (sa * sw[j]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < MS; ++i)
#pragma unroll
          for (int j = 0; j < NS; ++j) acc[i][j] = mfma_fp8_16x16x128(af[i], bf[j], acc[i][j]);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        v8s af[MS], bf[NS];
#pragma unroll
        for (int i = 0; i < MS; ++i)
          af[i] = *(const v8s*)(sA + (wm * WTM + i * 16 + l16) * LDR + lg * 64 + s * 16);
#pragma unroll
        for (int j = 0; j < NS; ++j)
          bf[j] = *(const v8s*)(sB + (wn * WTN + j * 16 + l16) * LDR + lg * 64 + s * 16);
#pragma unroll
        for (int i = 0; i < MS; ++i)
#pragma unroll
          for (int j = 0; j < NS; ++j) acc[i][j] = mfma_h16<DT>(af[i], bf[j], acc[i][j]);
      }
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogue
  uint16_t* C = (uint16_t*)p.C;
#pragma unroll
  for (int i = 0; i < MS; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tr = wm * WTM + i * 16 + lg * 4 + r;
      const int slot = sSlot[tr];
      if (slot < 0) continue;
      if constexpr (EPI == EPI_ACT) {
#pragma unroll
        for (int j = 0; j < NS / 2; ++j) {
          const int gcol = nt * (BN / 2) + wn * (WTN / 2) + j * 16 + l16;
          if (gcol >= p.inter) continue;
          const float g = round_h16<DT>(acc[i][j][r]);
          const float u = round_h16<DT>(acc[i][j + NS / 2][r]);
          const float a = round_h16<DT>(p.activation == 0 ? act_f32<0>(g) : act_f32<1>(g));
          C[(int64_t)slot * p.ldc + gcol] = f32_to_h16<DT>(a * u);
        }
      } else if constexpr (EPI == EPI_DENSE) {
        const float sa = p.a_scale[slot];
#pragma unroll
        for (int j = 0; j < NS; ++j) {
          const int col = nt * BN + wn * WTN + j * 16 + l16;
          if (col >= p.N) continue;
          const float v = acc[i][j][r] * sa * ((const float*)p.b_scale)[col];
          C[(int64_t)slot * p.ldc + col] = f32_to_h16<DT>(v);
        }
      } else {
        const float rw = p.mul_routed ? load_weight(p.topk_w, p.topk_w_dtype, slot) : 1.f;
#pragma unroll
        for (int j = 0; j < NS; ++j) {
          const int col = nt * BN + wn * WTN + j * 16 + l16;
          if (col >= p.N) continue;
          C[(int64_t)slot * p.ldc + col] = f32_to_h16<DT>(acc[i][j][r] * rw);
        }
      }
    }
  }
}

template <int AK, int BK, int EPI, int DT, bool GROUPED, int BM, int BN>
static int run_tile(const GemmArgs& a, hipStream_t stream) {
  using En = Engine<AK, BK>;
  const size_t shmem = (size_t)(BM + BN) * En::kLdr + BM * sizeof(float) + 2 * BM * sizeof(int);
  auto kern = tile_gemm_kernel<AK, BK, EPI, DT, GROUPED, BM, BN>;
  const int st = ensure_dynamic_lds((const void*)kern, shmem, "tile_gemm");
  if (st != kOk) return st;
  const int n_tiles = (EPI == EPI_ACT) ? (a.inter + BN / 2 - 1) / (BN / 2) : (a.N + BN - 1) / BN;
  const int64_t m_blocks = GROUPED ? a.m_blocks : (a.M + BM - 1) / BM;
  if (m_blocks == 0) return kOk;
  const int64_t grid = m_blocks * n_tiles;
  if (grid >= ((int64_t)1 << 31)) {
    set_last_error("tile_gemm: grid too large");
    return kUnsupported;
  }
  kern<<<dim3((unsigned)grid), dim3(256), shmem, stream>>>(a);
  return launch_status("tile_gemm");
}

template <int AK, int BK, int EPI, int DT, bool GROUPED>
static int dispatch_bm(const GemmArgs& a, int bm, hipStream_t s) {
  switch (bm) {
    case 16:
      if constexpr (AK == A_H16 && BK == B_H16) return run_tile<AK, BK, EPI, DT, GROUPED, 16, 128>(a, s);
      break;
    case 32: return run_tile<AK, BK, EPI, DT, GROUPED, 32, 128>(a, s);
    case 64: return run_tile<AK, BK, EPI, DT, GROUPED, 64, 128>(a, s);
    case 128: return run_tile<AK, BK, EPI, DT, GROUPED, 128, 128>(a, s);
  }
  set_last_error("tile_gemm: unsupported block size %d for this operand combination", bm);
  return kUnsupported;
}

int launch_tile_gemm(const GemmArgs& a, int akind, int bkind, int epi, int dtype, bool grouped,
                     int bm, hipStream_t stream) {
  const bool any_k = akind == A_H16 && bkind == B_H16;
  if (a.K <= 0 || (!any_k && a.K % 128 != 0) || a.N <= 0 || (epi == EPI_ACT && a.N != 2 * a.inter)) {
    set_last_error("tile_gemm: K must be positive (a multiple of 128 for quantised operands; "
                   "K=%d, N=%d)", a.K, a.N);
    return kInvalidArgument;
  }
  if (grouped && (!a.sorted_ids || !a.expert_ids || !a.ntpp)) {
    set_last_error("tile_gemm: grouped mode needs sorted_ids/expert_ids/ntpp");
    return kInvalidArgument;
  }
  if (akind == A_H16 && bkind == B_H16 && grouped) {
    if (dtype == kBF16) {
      if (epi == EPI_STORE) return dispatch_bm<A_H16, B_H16, EPI_STORE, kBF16, true>(a, bm, stream);
      if (epi == EPI_ACT) return dispatch_bm<A_H16, B_H16, EPI_ACT, kBF16, true>(a, bm, stream);
    } else if (dtype == kF16) {
      if (epi == EPI_STORE) return dispatch_bm<A_H16, B_H16, EPI_STORE, kF16, true>(a, bm, stream);
      if (epi == EPI_ACT) return dispatch_bm<A_H16, B_H16, EPI_ACT, kF16, true>(a, bm, stream);
    }
  } else if (akind == A_H16 && bkind == B_INT4G && grouped && dtype == kBF16) {
    if (epi == EPI_STORE) return dispatch_bm<A_H16, B_INT4G, EPI_STORE, kBF16, true>(a, bm, stream);
    if (epi == EPI_ACT) return dispatch_bm<A_H16, B_INT4G, EPI_ACT, kBF16, true>(a, bm, stream);
  } else if (akind == A_FP8G && bkind == B_FP8BLK && grouped && dtype == kBF16 && bm == kBigBlockM) {
    return launch_gemm_fp8_big(a, epi, true, kBigBlockM, stream);
  } else if (akind == A_FP8R && bkind == B_FP8R && !grouped && dtype == kBF16 && bm == kBigBlockM) {
    return launch_gemm_fp8_big(a, epi, false, kBigBlockM, stream);
  } else if (akind == A_FP8G && bkind == B_FP8BLK && grouped && dtype == kBF16) {
    if (epi == EPI_STORE) return dispatch_bm<A_FP8G, B_FP8BLK, EPI_STORE, kBF16, true>(a, bm, stream);
    if (epi == EPI_ACT) return dispatch_bm<A_FP8G, B_FP8BLK, EPI_ACT, kBF16, true>(a, bm, stream);
  } else if (akind == A_FP8R && bkind == B_FP8R && !grouped && dtype == kBF16 && epi == EPI_DENSE) {
    return dispatch_bm<A_FP8R, B_FP8R, EPI_DENSE, kBF16, false>(a, bm, stream);
  }
  set_last_error("tile_gemm: unsupported operand combination (A=%d B=%d epi=%d dtype=%d grouped=%d)",
                 akind, bkind, epi, dtype, (int)grouped);
  return kUnsupported;
}

// ---------------------------------------------------------------------------
// Weight-streaming grouped GEMM
// ---------------------------------------------------------------------------
// Rows of A staged per pass (LDS budget ~64 KB at K = 2048).
template <int BK>
struct StreamCfg {
  static constexpr bool kFp8 = BK == B_FP8BLK;
  static constexpr int kPassRows = kFp8 ? 32 : 16;
};

template <int BK, int EPI, int DT, int KS>
__global__ __launch_bounds__(256) void stream_gemm_kernel(GemmArgs p) {
  constexpr bool FP8 = StreamCfg<BK>::kFp8;
  constexpr int PR = StreamCfg<BK>::kPassRows;
  constexpr int K = KS * 128;
  constexpr int LDA = FP8 ? K + 16 : 2 * K + 16;  // LDS row stride (bytes)
  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* sA = smem;
  float* sAs = (float*)(sA + PR * LDA);  // FP8: [PR][KS] group scales
  __shared__ int sArow[PR];              // A row of each staged slot

  const int e = blockIdx.y, nt = blockIdx.x;
  const int cnt = p.expert_cnt[e];
  if (cnt == 0) return;
  const int off = p.expert_off[e];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;

  // Weight row feeding this lane's MFMA column.
  int brow, ocol;
  bool bvalid;
  if constexpr (EPI == EPI_ACT) {
    ocol = nt * 32 + w * 8 + (l16 & 7);
    bvalid = ocol < p.inter;
    brow = l16 < 8 ? ocol : p.inter + ocol;
  } else {
    ocol = nt * 64 + w * 16 + l16;
    bvalid = ocol < p.N;
    brow = ocol;
  }

  // Issue every weight load of this lane first.
  using BFrag = typename std::conditional<FP8, v8i, v4i>::type;
  BFrag bq[KS];
  float bsc[KS];
  if constexpr (FP8) {
    const uint8_t* src = (const uint8_t*)p.B + (int64_t)e * p.b_estride + (int64_t)brow * p.ldb + lg * 32;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      bq[kk] = bvalid ? *(const v8i*)(src + kk * 128) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
    const float* ss = (const float*)p.b_scale + (int64_t)e * p.bs_estride + (int64_t)(brow / 128) * p.bs_ld;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) bsc[kk] = bvalid ? ss[kk] : 0.f;
  } else {
    const int32_t* src = (const int32_t*)p.B + (int64_t)e * p.b_estride + (int64_t)brow * p.ldb + lg * 4;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      bq[kk] = bvalid ? *(const v4i*)(src + kk * 16) : v4i{0, 0, 0, 0};
    const uint16_t* ss = (const uint16_t*)p.b_scale + (int64_t)e * p.bs_estride + (int64_t)brow * p.bs_ld;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) bsc[kk] = bvalid ? h16_to_f32<DT>(ss[kk]) : 0.f;
  }

  const uint16_t* A16 = (const uint16_t*)p.A;
  for (int r0 = 0; r0 < cnt; r0 += PR) {
    const int rows = cnt - r0 < PR ? cnt - r0 : PR;
    if (r0 > 0) __syncthreads();
    // ---- stage A rows [r0, r0 + rows) into LDS
    if constexpr (FP8) {
      // 16 lanes per 128-element group; quantise as quant_fp8_group_kernel.
      const int groups = rows * KS;
      for (int g0 = 0; g0 < groups; g0 += 16) {
        const int g = g0 + (tid >> 4), sub = tid & 15;
        const bool live = g < groups;
        const int rr = live ? g / KS : 0, kk = live ? g % KS : 0;
        int arow = 0;
        if (live) arow = p.sorted_ids[off + r0 + rr] / p.top_k;
        v4i raw = live ? *(const v4i*)(A16 + (int64_t)arow * p.lda + kk * 128 + sub * 8)
                       : v4i{0, 0, 0, 0};
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f[2 * i] = h16_to_f32<DT>((uint16_t)(raw[i] & 0xffff));
          f[2 * i + 1] = h16_to_f32<DT>((uint16_t)((uint32_t)raw[i] >> 16));
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
          if (sub == 0) sAs[rr * KS + kk] = sc;
        }
      }
    } else {
      // Row indices first, then eight independent 16-byte loads per thread
      // in flight (one memory round trip per batch, not per chunk).
      if (tid < rows) sArow[tid] = p.sorted_ids[off + r0 + tid] / p.top_k;
      __syncthreads();
      const int chunks = rows * (K / 8);  // 16-byte chunks
      constexpr int kB = 8;
      for (int c0 = 0; c0 < chunks; c0 += 256 * kB) {
        v4i v[kB];
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          const int c = c0 + j * 256 + tid;
          const int rr = c / (K / 8), cc = c % (K / 8);
          v[j] = c < chunks ? *(const v4i*)(A16 + (int64_t)sArow[rr] * p.lda + cc * 8) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          const int c = c0 + j * 256 + tid;
          if (c < chunks) *(v4i*)(sA + (c / (K / 8)) * LDA + (c % (K / 8)) * 16) = v[j];
        }
      }
    }
    __syncthreads();

    // ---- MFMA over K for each 16-row group of this pass
    constexpr int MC = PR / 16;
    v4f acc[MC];
#pragma unroll
    for (int mc = 0; mc < MC; ++mc) acc[mc] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
      for (int mc = 0; mc < MC; ++mc) {
        if (mc * 16 >= rows) break;
        const int ar = mc * 16 + l16;
        if constexpr (FP8) {
          v8i af = ar < rows ? load_v8i_a16(sA + ar * LDA + kk * 128 + lg * 32)
                             : v8i{0, 0, 0, 0, 0, 0, 0, 0};
          v4f t = mfma_fp8_16x16x128(af, bq[kk], v4f{0.f, 0.f, 0.f, 0.f});
          v4f sa;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int orow = mc * 16 + lg * 4 + r;
            sa[r] = orow < rows ? sAs[orow * KS + kk] : 0.f;
          }
          acc[mc] += t * (sa * bsc[kk]);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            v8s af = ar < rows ? *(const v8s*)(sA + ar * LDA + (kk * 128 + lg * 32 + s * 8) * 2)
                               : v8s{0, 0, 0, 0, 0, 0, 0, 0};
            v8s bf = dequant_int4x8<DT>((uint32_t)bq[kk][s], bsc[kk]);
            acc[mc] = mfma_h16<DT>(af, bf, acc[mc]);
          }
        }
      }
    }

    // ---- epilogue
    uint16_t* C = (uint16_t*)p.C;
#pragma unroll
    for (int mc = 0; mc < MC; ++mc) {
      if (mc * 16 >= rows) break;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int orow = mc * 16 + lg * 4 + r;
        const float mine = acc[mc][r];
        if constexpr (EPI == EPI_ACT) {
          const float up = __shfl_xor(mine, 8, 64);
          if (orow < rows && l16 < 8 && bvalid) {
            const int slot = p.sorted_ids[off + r0 + orow];
            const float g = round_h16<DT>(mine);
            const float u = round_h16<DT>(up);
            const float a = round_h16<DT>(p.activation == 0 ? act_f32<0>(g) : act_f32<1>(g));
            C[(int64_t)slot * p.ldc + ocol] = f32_to_h16<DT>(a * u);
          }
        } else {
          if (orow < rows && bvalid) {
            const int slot = p.sorted_ids[off + r0 + orow];
            const float rw = p.mul_routed ? load_weight(p.topk_w, p.topk_w_dtype, slot) : 1.f;
            C[(int64_t)slot * p.ldc + ocol] = f32_to_h16<DT>(mine * rw);
          }
        }
      }
    }
  }
}

template <int BK, int EPI, int KS>
static int run_stream(const GemmArgs& a, hipStream_t stream) {
  constexpr bool FP8 = StreamCfg<BK>::kFp8;
  constexpr int PR = StreamCfg<BK>::kPassRows;
  constexpr int K = KS * 128;
  const size_t shmem = (size_t)PR * (FP8 ? K + 16 : 2 * K + 16) + (FP8 ? PR * KS * sizeof(float) : 0);
  auto kern = stream_gemm_kernel<BK, EPI, kBF16, KS>;
  const int st = ensure_dynamic_lds((const void*)kern, shmem, "stream_gemm");
  if (st != kOk) return st;
  const int n_tiles = EPI == EPI_ACT ? (a.inter + 31) / 32 : (a.N + 63) / 64;
  kern<<<dim3(n_tiles, a.num_experts), dim3(256), shmem, stream>>>(a);
  return launch_status("stream_gemm");
}

template <int BK, int EPI>
static int dispatch_ks(const GemmArgs& a, hipStream_t s) {
  switch (a.K / 128) {
    case 1: return run_stream<BK, EPI, 1>(a, s);
    case 2: return run_stream<BK, EPI, 2>(a, s);
    case 3: return run_stream<BK, EPI, 3>(a, s);
    case 4: return run_stream<BK, EPI, 4>(a, s);
    case 6: return run_stream<BK, EPI, 6>(a, s);
    case 8: return run_stream<BK, EPI, 8>(a, s);
    case 12: return run_stream<BK, EPI, 12>(a, s);
    case 16: return run_stream<BK, EPI, 16>(a, s);
  }
  set_last_error("stream_gemm: unsupported K=%d", a.K);
  return kUnsupported;
}

// The decode path is bound by HBM, not by the MFMA rate, so it reduces the
// FP8 products with the fp32-exact bf16 MFMA (see block_dot_fp8).
constexpr bool kStreamExact = true;

bool stream_gemm_supported(int K, int max_rows, int akind, int bkind) {
  (void)max_rows;
  if (K % 128 != 0) return false;
  const int ks = K / 128;
  const bool ks_ok = ks == 1 || ks == 2 || ks == 3 || ks == 4 || ks == 6 || ks == 8 || ks == 12 || ks == 16;
  return ks_ok && akind == A_H16 && (bkind == B_FP8BLK || bkind == B_INT4G);
}

int launch_stream_gemm(const GemmArgs& a, int akind, int bkind, int epi, int dtype, int max_rows,
                       hipStream_t stream) {
  if (!stream_gemm_supported(a.K, max_rows, akind, bkind) || dtype != kBF16) {
    set_last_error("stream_gemm: unsupported configuration (K=%d A=%d B=%d dtype=%d)", a.K, akind,
                   bkind, dtype);
    return kUnsupported;
  }
  if ((!a.topk_ids && (!a.expert_off || !a.expert_cnt || !a.sorted_ids)) ||
      (epi == EPI_ACT && a.N != 2 * a.inter)) {
    set_last_error("stream_gemm: missing expert offsets/counts or bad shapes");
    return kInvalidArgument;
  }
  if (bkind == B_FP8BLK) return launch_stream_fp8(a, epi, kStreamExact, stream);
  if (a.topk_ids) return launch_stream_int4_cu(a, epi, stream);
  return epi == EPI_ACT ? dispatch_ks<B_INT4G, EPI_ACT>(a, stream)
                        : dispatch_ks<B_INT4G, EPI_STORE>(a, stream);
}

}  // namespace mstar
