// Tiled grouped GEMM for W4A16 MoE layers above decode size: int4 weights
// (group-128 bf16 scales whose products with the codes are exact in bf16)
// times bf16 token rows, for the reference's fused_moe_kernel contract
// (mstar/utils/fused_moe/kernels.py:83-138: one block of sorted_ids per
// tile row, A row = slot / top_k, padding masked, blocks past
// num_tokens_post_padded skipped) with the activation or routed-weight
// epilogues of fused_experts (runner.py:99-159).
//
// Tile: 64 tokens (one alignment block) x 256 weight rows, 8 waves; wave w
// owns all 64 tokens x 32 weight rows (two 16-row subtiles).  K is walked in
// steps of 256 (two scale groups): per step the 64 token rows (32 KB bf16),
// the 256 weight rows (one whole 128-byte line each, 32 KB int4), the rows'
// scales and the tokens' group sums go from global memory to LDS by LDS-DMA
// (global_load_lds) into a two-stage ring; the next step loads while this
// one computes, one barrier per step.  Persistent over tiles.
//
// Math (no dequantisation pass): a code pair becomes the bf16 pair
// 0x4300|u = 128 + u with one v_bfi_b32, bf16 MFMAs (weights as the A
// operand, tokens as B) sum (128 + u) x over a group, and
//   sum (u - 8) s x = s (t - 136 sum x)
// recovers the group's contribution of the bf16 weights q * s exactly up
// to fp32 rounding (sum x is precomputed per token row and group).  The
// codes unpack in the pair order 0, 4, 1, 5, 2, 6, 3, 7 of each 8-group,
// so token rows are stored in that order: w4_prep_kernel writes the hidden
// rows so, and the gate_up epilogue writes its activation output so (by
// loading weight rows in that order), together with the group sums the
// down GEMM needs.  No operand is permuted in the main loop.
#include "common.h"
#include "launch.h"

namespace mstar {

constexpr int kW4BM = 64, kW4BN = 256, kW4Threads = 512;
constexpr int kW4TokBytes = kW4BM * 512;           // 64 rows x 256 K bf16
constexpr int kW4WBytes = kW4BN * 128;             // 256 rows x 256 K int4
constexpr int kW4ScOff = kW4TokBytes + kW4WBytes;  // row scales [256][2] bf16
constexpr int kW4XOff = kW4ScOff + kW4BN * 4;      // token group sums [64][2] fp32
constexpr int kW4Stage = kW4XOff + kW4BM * 8;
constexpr int kW4IdBufs = 4;
constexpr int kW4Lds = 2 * kW4Stage + kW4IdBufs * kW4BM * 4 + 8 * kW4BM * 4;  // + ids, group-sum partials

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// Token-row chunk swizzle: a row's 16-byte piece l is stored at position
// l ^ w4_tok_swz(row % 16).  A ds_read_b128 is served in four passes of 16
// lanes, and the lanes of one pass are a coset of the lane-index subspace
// spanned by 1, 2, 12 and 24 (measured with mstar_amd/microbench/lds_banks.hip).
// The fragment read of lane (l16, lg) takes piece 4 lg + kc of row
// 16 i + l16; with this swizzle the 16 lanes of every pass land on 16
// different bank quads.  (Plain l ^ row is conflict-free for
// 16 consecutive lanes but two-way conflicted on these passes.)
__device__ __forceinline__ int w4_tok_swz(int r) { return r ^ (((r >> 2) & 1) << 3); }

// Logical column (element) at stored position p of a 16-wide segment: each
// 8-group holds elements 0, 4, 1, 5, 2, 6, 3, 7.
__device__ __forceinline__ int w4_pair_elem(int p) { return (p & 8) | ((p & 1) << 2) | ((p >> 1) & 3); }

// Hidden rows in pair order plus their per-128-group fp32 sums.  One lane
// per 8 elements; the 16 lanes of a group are one DPP row.
__global__ __launch_bounds__(256) void w4_prep_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                      int64_t rows, int H, uint16_t* __restrict__ out,
                                                      float* __restrict__ xs) {
  const int64_t per_row = H / 8;
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool live = v < rows * per_row;
  const int64_t r = live ? v / per_row : 0, c8 = live ? v % per_row : 0;
  const v4i d = live ? *(const v4i*)(x + r * ldx + c8 * 8) : v4i{0, 0, 0, 0};
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = (uint32_t)d[i];
    sum += bf16_bits_to_f32((uint16_t)(w & 0xffffu)) + bf16_bits_to_f32((uint16_t)(w >> 16));
  }
  sum = row_fsum16(sum);
  if (!live) return;
  const uint32_t d0 = d[0], d1 = d[1], d2 = d[2], d3 = d[3];
  *(v4i*)(out + r * H + c8 * 8) =
      v4i{(int)((d0 & 0xffffu) | (d2 << 16)), (int)((d0 >> 16) | (d2 & 0xffff0000u)),
          (int)((d1 & 0xffffu) | (d3 << 16)), (int)((d1 >> 16) | (d3 & 0xffff0000u))};
  if ((c8 & 15) == 0) xs[r * (H / 128) + c8 / 16] = sum;
}

// EPI_ACT: gate_up with SiLU/GeLU-and-mul; C [slots, inter] bf16 in pair
// order and xs_out [slots, inter / 128] the group sums of the stored values.
// EPI_STORE: down times the routed weight into C [slots, N] (natural order).
// xs: group sums of the A rows [rows, K / 128].
//
// Persistent: one workgroup per CU walks tiles (m-block major; within a
// round the workgroups of an XCD take consecutive tiles, so an m-block's
// n-tiles share token rows in one L2).  The DMA runs one step ahead across
// tile boundaries: the next tile's first step loads during this tile's
// last step and epilogue; each tile's sorted_ids block arrives by DMA three
// tiles ahead, into one of four LDS buffers.
template <int EPI>
__global__ __launch_bounds__(kW4Threads) void w4_tile_kernel(GemmArgs p, const float* __restrict__ xs,
                                                             float* __restrict__ xs_out) {
  extern __shared__ __align__(16) uint8_t smem[];
  int* sIds = (int*)(smem + 2 * kW4Stage);             // [4][64] sorted_ids blocks
  float* sPart = (float*)(sIds + kW4IdBufs * kW4BM);  // [8 waves][64 tokens]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int n_tiles = EPI == EPI_ACT ? p.inter / 128 : p.N / kW4BN;
  typedef const __attribute__((address_space(4))) int* const_iptr;
  const int m_valid = (((const_iptr)p.ntpp)[0] + kW4BM - 1) / kW4BM;
  const int total = m_valid * n_tiles;
  const int G = gridDim.x;
  auto tile_of = [&](int j) -> int {
    const int r = (G % 8 == 0) ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    return j * G + r;
  };
  if (tile_of(0) >= total) return;
  const int KG = p.K / 128;  // scale groups along K
  const int steps = p.K / 256;

  // sorted_ids block of tile t into buffer b (wave 0, one dword per lane).
  auto issue_ids = [&](int t, int b) {
    if (t < total && wave == 0)
      __builtin_amdgcn_global_load_lds((const void*)(p.sorted_ids + (int64_t)(t / n_tiles) * kW4BM + lane),
                                       (lds_void_ptr)(sIds + b * kW4BM), 4, 0, 0);
  };
  auto slot_of = [&](int b, int tok) -> int {
    const int s = sIds[b * kW4BM + tok];
    return s < p.M ? s : -1;
  };

  // ---- DMA of a step into a stage.  Tokens: instruction q of wave w
  // fills rows 8w + 2q + (lane / 32), physical piece lane % 32 holding
  // logical piece (lane % 32) ^ w4_tok_swz(row % 16).  Weights: instruction q of wave
  // w fills rows 32w + 8q + lane / 8, physical piece lane % 8 holding
  // logical piece (lane % 8) ^ ((row / 2) % 8).  Waves 0-3: the scales of
  // rows 64w + lane; waves 4-5: the token group sums.  setup() points the
  // sources at tile t (ids in buffer b).
  const uint8_t* a_src[4];
  const uint8_t* w_src[4];
  const uint8_t* aux_src = nullptr;
  auto setup = [&](int t, int b) {
    const int mb = t / n_tiles, nt = t % n_tiles;
    const int expert = __builtin_amdgcn_readfirstlane(((const_iptr)p.expert_ids)[mb]);
    // Global weight row of LDS row rho.  Activation: wave column w's rows
    // are 16 gate rows then the 16 matching up rows of act columns
    // nt * 128 + 16 w + [0, 16), taken in pair order.
    auto grow = [&](int rho) -> int {
      if constexpr (EPI == EPI_ACT) {
        const int wv = rho >> 5, qq = rho & 31;
        const int col = nt * 128 + 16 * wv + w4_pair_elem(qq & 15);
        return qq < 16 ? col : p.inter + col;
      } else {
        return nt * kW4BN + rho;
      }
    };
    auto arow_of = [&](int tok) -> int {
      const int s = slot_of(b, tok);
      return s < 0 ? 0 : s / p.top_k;
    };
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int tok = 8 * wave + 2 * q + (lane >> 5);
      const int lp = (lane & 31) ^ w4_tok_swz(tok & 15);
      a_src[q] = (const uint8_t*)p.A + ((int64_t)arow_of(tok) * p.lda) * 2 + lp * 16;
      const int rho = 32 * wave + 8 * q + (lane >> 3);
      const int wp = (lane & 7) ^ ((rho >> 1) & 7);
      w_src[q] = (const uint8_t*)((const int32_t*)p.B + (int64_t)expert * p.b_estride +
                                  (int64_t)grow(rho) * p.ldb) + wp * 16;
    }
    if (wave < 4) {
      aux_src = (const uint8_t*)((const uint16_t*)p.b_scale + (int64_t)expert * p.bs_estride +
                                 (int64_t)grow(64 * wave + lane) * p.bs_ld);
    } else if (wave < 6) {
      const int idx = (wave - 4) * 64 + lane;
      aux_src = (const uint8_t*)(xs + (int64_t)arow_of(idx >> 1) * KG + (idx & 1));
    }
  };
  auto issue = [&](int st, int sg) {
    uint8_t* base = smem + sg * kW4Stage;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      __builtin_amdgcn_global_load_lds((const void*)(a_src[q] + st * 512),
                                       (lds_void_ptr)(base + (8 * wave + 2 * q) * 512), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(w_src[q] + st * 128),
                                       (lds_void_ptr)(base + kW4TokBytes + (32 * wave + 8 * q) * 128), 16, 0, 0);
    }
    if (wave < 4)
      __builtin_amdgcn_global_load_lds((const void*)(aux_src + st * 4),
                                       (lds_void_ptr)(base + kW4ScOff + wave * 256), 4, 0, 0);
    else if (wave < 6)
      __builtin_amdgcn_global_load_lds((const void*)(aux_src + st * 8),
                                       (lds_void_ptr)(base + kW4XOff + (wave - 4) * 256), 4, 0, 0);
  };

  // Prologue: ids of tiles 0-2, then tile 0's first step.
  issue_ids(tile_of(0), 0);
  issue_ids(tile_of(1), 1);
  wait_vmcnt<0>();
  __syncthreads();
  setup(tile_of(0), 0);
  issue(0, 0);
  issue_ids(tile_of(2), 2);

  const Int4BiasConsts k4 = int4_bias_consts();
  uint16_t* C = (uint16_t*)p.C;
  int qs = 0;  // global step: ring stage qs & 1
  for (int j = 0; tile_of(j) < total; ++j) {
    const int nt = tile_of(j) % n_tiles, buf = j % kW4IdBufs;
    v4f acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) acc[i][jj] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int st = 0; st < steps; ++st, ++qs) {
      wait_vmcnt<0>();
      lds_barrier();  // the step landed for every wave; every wave is past the previous one
      if (st + 1 < steps) {
        issue(st + 1, (qs + 1) & 1);
      } else if (tile_of(j + 1) < total) {  // the next tile's first step
        setup(tile_of(j + 1), (j + 1) % kW4IdBufs);
        issue(0, (qs + 1) & 1);
        issue_ids(tile_of(j + 3), (j + 3) % kW4IdBufs);
      }
      const uint8_t* base = smem + (qs & 1) * kW4Stage;
      const uint8_t* sTok = base;
      const uint8_t* sW = base + kW4TokBytes;
      // Scales of this lane's rows 4 lg + r of both subtiles, both groups.
      v4i sc[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) sc[jj] = *(const v4i*)(base + kW4ScOff + (32 * wave + 16 * jj + 4 * lg) * 4);
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        v4i wq[2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int rho = 32 * wave + 16 * jj + l16;
          wq[jj] = *(const v4i*)(sW + rho * 128 + (((g * 4 + lg) ^ ((l16 >> 1) & 7)) << 4));
        }
        v4f t[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) t[i][jj] = v4f{0.f, 0.f, 0.f, 0.f};
        // Token fragments one K-chunk ahead: the reads of chunk kc + 1 are
        // in flight while chunk kc's MFMAs run.
        auto tok_frag = [&](int i, int kc) -> v8s {
          return *(const v8s*)(sTok + (16 * i + l16) * 512 + (((g * 16 + lg * 4 + kc) ^ w4_tok_swz(l16)) << 4));
        };
        v8s bcur[4], bnxt[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) bcur[i] = tok_frag(i, 0);
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
          if (kc + 1 < 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) bnxt[i] = tok_frag(i, kc + 1);
          }
          __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of this chunk's MFMAs
          v8s a[2];
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) a[jj] = int4x8_bias128((uint32_t)wq[jj][kc], k4);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) t[i][jj] = mfma_bf16_16x16x32(a[jj], bcur[i], t[i][jj]);
          __builtin_amdgcn_sched_barrier(0);
          if (kc + 1 < 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) bcur[i] = bnxt[i];
          }
        }
        // s (t - 136 sum x) per (row, token): rows 4 lg + r, token 16 i + l16.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float bias = -136.f * ((const float*)(base + kW4XOff))[(16 * i + l16) * 2 + g];
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const uint32_t two = (uint32_t)sc[jj][r];
              const float s = bf16_bits_to_f32((uint16_t)(g == 0 ? two & 0xffffu : two >> 16));
              acc[i][jj][r] = __builtin_fmaf(t[i][jj][r] + bias, s, acc[i][jj][r]);
            }
        }
      }
    }

    // ---- epilogue: lane (l16, lg) holds rows 4 lg + r of subtiles jj for
    // tokens 16 i + l16.  The next tile's first step is in flight.
    if constexpr (EPI == EPI_ACT) {
      // a = bf16(bf16(act(bf16(gate))) * bf16(up)) (kernels.py:279-298),
      // stored at position 4 lg + r of the wave's 16-column segment (pair
      // order by construction of the weight rows).
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = 16 * i + l16, slot = slot_of(buf, tok);
        uint32_t pk[2];
        float psum = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint32_t two = 0;
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int r = 2 * h + e;
            const float gg = round_bf16(acc[i][0][r]);
            const float u = round_bf16(acc[i][1][r]);
            const float av = round_bf16(p.activation == 0 ? act_f32<0>(gg) : act_f32<1>(gg));
            const uint16_t y = f32_to_bf16_bits(av * u);
            psum += bf16_bits_to_f32(y);
            two |= (uint32_t)y << (16 * e);
          }
          pk[h] = two;
        }
        if (slot >= 0)
          *(uint2*)(C + (int64_t)slot * p.ldc + nt * 128 + 16 * wave + 4 * lg) = make_uint2(pk[0], pk[1]);
        psum += __shfl_xor(psum, 16, 64);
        psum += __shfl_xor(psum, 32, 64);
        if (lg == 0) sPart[wave * kW4BM + tok] = psum;
      }
      lds_sync();
      if (tid < kW4BM) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w) s += sPart[w * kW4BM + tid];
        const int slot = slot_of(buf, tid);
        if (slot >= 0) xs_out[(int64_t)slot * (p.inter / 128) + nt] = s;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = 16 * i + l16, slot = slot_of(buf, tok);
        if (slot < 0) continue;
        const float rw = p.mul_routed ? load_weight_any(p.topk_w, p.topk_w_dtype, slot) : 1.f;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const uint32_t lo = (uint32_t)f32_to_bf16_bits(acc[i][jj][0] * rw) |
                              ((uint32_t)f32_to_bf16_bits(acc[i][jj][1] * rw) << 16);
          const uint32_t hi = (uint32_t)f32_to_bf16_bits(acc[i][jj][2] * rw) |
                              ((uint32_t)f32_to_bf16_bits(acc[i][jj][3] * rw) << 16);
          *(uint2*)(C + (int64_t)slot * p.ldc + nt * kW4BN + 32 * wave + 16 * jj + 4 * lg) = make_uint2(lo, hi);
        }
      }
    }
  }
  wait_vmcnt<0>();  // no DMA outlives the kernel
}

bool w4_tile_supported(int64_t H, int64_t I) { return H % 256 == 0 && I % 256 == 0; }

int launch_w4_prep(const void* x, int64_t ldx, int64_t rows, int64_t H, void* out, float* xs,
                   hipStream_t stream) {
  if (rows < 0 || H <= 0 || H % 128 != 0) {
    set_last_error("w4_prep: hidden size must be a positive multiple of 128");
    return kInvalidArgument;
  }
  if (rows == 0) return kOk;
  const int64_t threads = rows * (H / 8);
  w4_prep_kernel<<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream>>>(
      (const uint16_t*)x, ldx, rows, (int)H, (uint16_t*)out, xs);
  return launch_status("w4_prep");
}

template <int EPI>
static int run_w4_tile(const GemmArgs& a, const float* xs, float* xs_out, hipStream_t stream) {
  auto kern = w4_tile_kernel<EPI>;
  const int st = ensure_dynamic_lds((const void*)kern, kW4Lds, "w4_tile");
  if (st != kOk) return st;
  // Persistent: one workgroup per CU (the LDS ring allows no more).
  const int cus = device_cu_count();
  if (cus <= 0) return kLaunchError;
  if (a.m_blocks == 0) return kOk;
  kern<<<dim3((unsigned)cus), dim3(kW4Threads), kW4Lds, stream>>>(a, xs, xs_out);
  return launch_status("w4_tile");
}

int launch_w4_tile(const GemmArgs& a, int epi, const float* xs, float* xs_out, hipStream_t stream) {
  if (a.K <= 0 || a.K % 256 != 0 || !xs ||
      (epi == EPI_ACT ? (a.inter % 128 != 0 || a.N != 2 * a.inter || !xs_out) : a.N % kW4BN != 0)) {
    set_last_error("w4_tile: needs K %% 256 == 0 and inter %% 128 == 0 (gate_up) or N %% 256 == 0 (down)");
    return kInvalidArgument;
  }
  if (epi == EPI_ACT) return run_w4_tile<EPI_ACT>(a, xs, xs_out, stream);
  if (epi == EPI_STORE) return run_w4_tile<EPI_STORE>(a, xs, xs_out, stream);
  set_last_error("w4_tile: unsupported epilogue %d", epi);
  return kUnsupported;
}

}  // namespace mstar
