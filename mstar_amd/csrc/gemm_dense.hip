// Dense W8A8 GEMM for decode-sized token counts (M <= 32): the per-token x
// per-channel FP8 scaled GEMM of the model's linear layers
// (out = (A_fp8 . W_fp8^T) * s_a[token] * s_w[channel], bf16), which at
// this size is a pure weight stream.
//
// Persistent: one 512-thread workgroup per CU takes an equal contiguous
// range of items (16 weight rows each).  The token rows (e4m3fn bytes),
// their scales and the range's channel scales are staged in LDS once; each
// wave then streams its items' weight rows through a private LDS ring (as
// many slots as the LDS allows, up to 8) with LDS-DMA loads (one
// instruction = 8 rows x one whole 128-byte line, the 16-byte pieces of row
// r stored at piece ^ (r % 8)), ring - 1 K-steps ahead of its MFMAs.  Each K-step of an item is one
// v_mfma_f32_16x16x128_f8f6f4 per 16 tokens, chained in the accumulator
// (no per-step scaling: the scales are per token and per channel).
// Token rows are stored with their 16-byte pieces at piece ^ (row % 16), so
// the 16 rows of an MFMA operand read fall in distinct banks.
#include "common.h"
#include "launch.h"

namespace mstar {

constexpr int kDsThreads = 512, kDsWaves = kDsThreads / 64;
constexpr int kDsStep = 16 * 128;  // bytes of one K-step of 16 rows
constexpr int kDsMaxTokens = 32;
constexpr size_t kDsLdsMax = 160 * 1024;

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// LDS: rings [8][RING][KC K-steps] | tokens [MS*16][K] (the scales are read
// from global memory).  Chunks of two K-steps halve the per-chunk overhead
// where the LDS allows three of them per wave; otherwise one K-step and a
// ring as deep as fits (the bytes in flight per wave hide HBM latency).
__host__ __device__ inline size_t ds_tok_off(int ring, int kc) { return (size_t)kDsWaves * ring * kc * kDsStep; }
__host__ __device__ inline size_t ds_lds_bytes(int ring, int kc, int64_t ms, int64_t K) {
  return ds_tok_off(ring, kc) + (size_t)ms * 16 * K;
}

// Wait for the oldest of `ahead` chunks (D DMA instructions each).
template <int N, int D>
__device__ __forceinline__ void ds_wait_oldest(int ahead) {
  if constexpr (N > 1) {
    if (ahead >= N) {
      wait_vmcnt<D * (N - 1)>();
      return;
    }
    ds_wait_oldest<N - 1, D>(ahead);
  } else {
    wait_vmcnt<0>();
  }
}

// MS token subtiles of 16, RING ring slots per wave, KC K-steps per slot.
template <int MS, int RING, int KC>
__global__ __launch_bounds__(kDsThreads) void dense_stream_kernel(GemmArgs p, int items_per_wg) {
  constexpr int kDsRing = RING, kDsSlot = KC * kDsStep;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int K = p.K, KS = K / 128;
  const int items = p.N / 16;
  const int i0 = blockIdx.x * items_per_wg;
  const int i1 = i0 + items_per_wg < items ? i0 + items_per_wg : items;
  if (i0 >= i1) return;
  uint8_t* ring = smem + (size_t)w * kDsRing * kDsSlot;
  uint8_t* sTok = smem + ds_tok_off(RING, KC);
  const uint8_t* A = (const uint8_t*)p.A;
  const uint8_t* B = (const uint8_t*)p.B;
  const float* bsc = (const float*)p.b_scale;

  // ---- staging: token rows by LDS-DMA (1 KB = 64 pieces per instruction;
  // rows past M read row 0), token scales, the range's channel scales.
  {
    const int ppr = K / 16;                 // pieces per row
    const int total = MS * 16 * ppr;        // pieces, a multiple of 64
    for (int b0 = w * 64; b0 < total; b0 += kDsThreads) {
      const int pc = b0 + lane, row = pc / ppr, phys = pc - row * ppr;
      const int logical = phys ^ (row & 15);
      const int arow = row < p.M ? row : 0;
      __builtin_amdgcn_global_load_lds((const void*)(A + (int64_t)arow * p.lda + logical * 16),
                                       (lds_void_ptr)(sTok + (size_t)b0 * 16), 16, 0, 0);
    }
  }
  // This lane's token scales (tokens 16 i + l16).
  float sa[MS];
#pragma unroll
  for (int i = 0; i < MS; ++i) sa[i] = 16 * i + l16 < p.M ? p.a_scale[16 * i + l16] : 0.f;

  // ---- the wave's chunks: item it = i0 + w + 8k, K-step c.
  const int r8 = lane >> 3;
  const uint32_t lc16 = (uint32_t)(((lane & 7) ^ r8) * 16);
  // K-step h of a chunk: rows 0-7 at 2h KB, rows 8-15 at (2h + 1) KB.
  auto dma = [&](int it, int c, int slot) {
    uint8_t* dst = ring + slot * kDsSlot;
#pragma unroll
    for (int h = 0; h < KC; ++h) {
      const uint8_t* src = B + (int64_t)(it * 16 + r8) * p.ldb + (c * KC + h) * 128 + lc16;
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void_ptr)(dst + 2 * h * 1024), 16, 0, 2);
      __builtin_amdgcn_global_load_lds((const void*)(src + 8 * p.ldb), (lds_void_ptr)(dst + (2 * h + 1) * 1024),
                                       16, 0, 2);
    }
  };
  int iit = i0 + w, ic = 0, islot = 0, ahead = 0;  // issue cursor
  auto issue_next = [&]() {
    dma(iit, ic, islot);
    islot = islot + 1 == kDsRing ? 0 : islot + 1;
    ++ahead;
    if (++ic == KS / KC) {
      ic = 0;
      iit += kDsWaves;
    }
  };
  while (iit < i1 && ahead < kDsRing - 1) issue_next();
  wait_vmcnt<0>();  // the staging loads (and the first chunks): one wait
  __syncthreads();

  uint16_t* C = (uint16_t*)p.C;
  int cslot = 0;
  for (int it = i0 + w; it < i1; it += kDsWaves) {
    v4f acc[MS];
#pragma unroll
    for (int i = 0; i < MS; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
    // This lane's channel scales, read now and used after the item.
    const v4f swv = *(const v4f*)(bsc + (int64_t)it * 16 + 4 * lg);
    for (int c = 0; c < KS / KC; ++c) {
      if (iit < i1) issue_next();
      // Wait for this chunk: the younger chunks (two instructions each) stay
      // in flight; epilogue stores between them only make this stricter.
      ds_wait_oldest<RING, 2 * KC>(ahead);
#pragma unroll
      for (int h = 0; h < KC; ++h) {
        const uint8_t* wrow = ring + cslot * kDsSlot + (2 * h + (l16 >> 3)) * 1024 + (l16 & 7) * 128;
        const int sw = l16 & 7;
        const v4i wlo = *(const v4i*)(wrow + (((2 * lg) ^ sw) << 4));
        const v4i whi = *(const v4i*)(wrow + (((2 * lg + 1) ^ sw) << 4));
        const v8i wf = v8i{wlo[0], wlo[1], wlo[2], wlo[3], whi[0], whi[1], whi[2], whi[3]};
#pragma unroll
        for (int i = 0; i < MS; ++i) {
          const int row = 16 * i + l16;
          const uint8_t* trow = sTok + (size_t)row * K;
          const int pc = (c * KC + h) * 8 + 2 * lg;
          const v4i tlo = *(const v4i*)(trow + ((pc ^ l16) << 4));
          const v4i thi = *(const v4i*)(trow + (((pc + 1) ^ l16) << 4));
          acc[i] = mfma_fp8_16x16x128(wf, v8i{tlo[0], tlo[1], tlo[2], tlo[3], thi[0], thi[1], thi[2], thi[3]},
                                      acc[i]);
        }
      }
      cslot = cslot + 1 == kDsRing ? 0 : cslot + 1;
      --ahead;
    }
    // Lane (l16, lg) holds channels it*16 + 4 lg + r for token 16 i + l16.
    const int n0 = it * 16 + 4 * lg;
#pragma unroll
    for (int i = 0; i < MS; ++i) {
      const int tok = 16 * i + l16;
      if (tok < p.M) {
        const uint32_t lo = (uint32_t)f32_to_bf16_bits(acc[i][0] * sa[i] * swv[0]) |
                            ((uint32_t)f32_to_bf16_bits(acc[i][1] * sa[i] * swv[1]) << 16);
        const uint32_t hi = (uint32_t)f32_to_bf16_bits(acc[i][2] * sa[i] * swv[2]) |
                            ((uint32_t)f32_to_bf16_bits(acc[i][3] * sa[i] * swv[3]) << 16);
        *(uint2*)(C + (int64_t)tok * p.ldc + n0) = make_uint2(lo, hi);
      }
    }
  }
  wait_vmcnt<0>();  // no DMA outlives the kernel
}


bool dense_stream_supported(int64_t M, int64_t N, int64_t K) {
  // K % 256: the token rows' pieces are swizzled within groups of 16.
  if (M <= 0 || M > kDsMaxTokens || N % 16 != 0 || K % 256 != 0 || K <= 0) return false;
  const int64_t ms = (M + 15) / 16;
  const int64_t items = N / 16;
  const int64_t per = (items + 255) / 256;  // worst case (at least 256 CUs)
  (void)per;
  return ds_lds_bytes(4, 1, ms, K) <= kDsLdsMax;
}

template <int MS, int RING, int KC>
static int run_dense_stream(const GemmArgs& a, hipStream_t stream) {
  const int cus = device_cu_count();
  if (cus <= 0) return kLaunchError;
  const int items = a.N / 16;
  const int per = (items + cus - 1) / cus;
  const size_t shmem = ds_lds_bytes(RING, KC, MS, a.K);
  if (shmem > kDsLdsMax) {
    set_last_error("dense_stream: %zu bytes of LDS needed", shmem);
    return kUnsupported;
  }
  auto kern = dense_stream_kernel<MS, RING, KC>;
  const int st = ensure_dynamic_lds((const void*)kern, shmem, "dense_stream");
  if (st != kOk) return st;
  kern<<<dim3((unsigned)cus), dim3(kDsThreads), shmem, stream>>>(a, per);
  return launch_status("dense_stream");
}

int launch_dense_stream(const GemmArgs& a, hipStream_t stream) {
  if (!dense_stream_supported(a.M, a.N, a.K) || a.ldc % 4 != 0) {
    set_last_error("dense_stream: unsupported shape (M=%lld N=%d K=%d)", (long long)a.M, a.N, a.K);
    return kUnsupported;
  }
  const int64_t ms = (a.M + 15) / 16;
  const bool two = a.K % 256 == 0 && ds_lds_bytes(3, 2, ms, a.K) <= kDsLdsMax;
  const bool mid = ds_lds_bytes(5, 1, ms, a.K) <= kDsLdsMax;
  if (ms == 1) return two ? run_dense_stream<1, 3, 2>(a, stream) : mid ? run_dense_stream<1, 5, 1>(a, stream)
                                                                : run_dense_stream<1, 4, 1>(a, stream);
  return two ? run_dense_stream<2, 3, 2>(a, stream) : mid ? run_dense_stream<2, 5, 1>(a, stream)
                                                  : run_dense_stream<2, 4, 1>(a, stream);
}

}  // namespace mstar
