// Activation quantisation to OCP e4m3fn for the W8A8 paths.
//
//  * per-token-group-128: s = max(amax, 1e-10) / 448, q = e4m3(clamp(x / s))
//    (the activation format of the block-scaled FP8 MoE GEMMs);
//  * per-row: one scale per token (the dense FP8 scaled GEMM).
// Division is IEEE (hipcc's default correctly-rounded fp32 divide) and the
// conversion is round-to-nearest-even, so the codes equal a CPU restatement
// bit for bit.
#include "common.h"
#include "launch.h"

namespace mstar {

// 16 lanes per 128-element group, 8 elements per lane.
// WIDEN: q holds the e4m3fn values widened to bf16 (2 bytes per element).
template <int DT, bool WIDEN>
__global__ __launch_bounds__(256) void quant_fp8_group_kernel(const uint16_t* __restrict__ x,
                                                              int64_t rows, int64_t cols,
                                                              int64_t ld_x, void* __restrict__ q,
                                                              float* __restrict__ s) {
  const int64_t gpr = cols / 128;
  const int64_t g = ((int64_t)blockIdx.x * 256 + threadIdx.x) / 16;
  const int sub = threadIdx.x & 15;
  const bool live = g < rows * gpr;
  const int64_t r = live ? g / gpr : 0, c = live ? (g % gpr) * 128 + sub * 8 : 0;
  v4i raw = live ? *(const v4i*)(x + r * ld_x + c) : v4i{0, 0, 0, 0};
  float sc;
  const int2 codes = quant_group8<DT>(raw, sc);
  if (live) {
    if constexpr (WIDEN)
      *(v4i*)((uint16_t*)q + r * cols + c) = fp8x8_to_bf16x8_bits(codes.x, codes.y);
    else
      *(int2*)((uint8_t*)q + r * cols + c) = codes;
    if (sub == 0) s[r * gpr + c / 128] = sc;
  }
}

// One workgroup per row.
template <int DT>
__global__ __launch_bounds__(256) void quant_fp8_row_kernel(const uint16_t* __restrict__ x,
                                                            int64_t cols,
                                                            uint8_t* __restrict__ q,
                                                            float* __restrict__ s) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const uint16_t* xr = x + r * cols;
  float amax = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) amax = fmaxf(amax, fabsf(h16_to_f32<DT>(xr[c])));
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = fmaxf(amax, kQuantEps) / kFp8Max;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    int v = cvt_pk_fp8<false>(clamp_fp8(h16_to_f32<DT>(xr[c]) / sc), 0.f, 0);
    q[r * cols + c] = (uint8_t)(v & 0xff);
  }
  if (threadIdx.x == 0) s[r] = sc;
}

int launch_quant_fp8_group(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ld_x,
                           void* q, float* s, hipStream_t stream, bool widen) {
  if (rows < 0 || cols <= 0 || cols % 128 != 0 || ld_x < cols || ld_x % 8 != 0) {
    set_last_error("quant_fp8_group: cols must be a positive multiple of 128 (cols=%lld)",
                   (long long)cols);
    return kInvalidArgument;
  }
  if (rows == 0) return kOk;
  const int64_t groups = rows * (cols / 128);
  dim3 grid((unsigned)((groups * 16 + 255) / 256));
  if (x_dtype == kBF16)
    widen ? quant_fp8_group_kernel<kBF16, true><<<grid, 256, 0, stream>>>((const uint16_t*)x, rows, cols, ld_x, q, s)
          : quant_fp8_group_kernel<kBF16, false><<<grid, 256, 0, stream>>>((const uint16_t*)x, rows, cols, ld_x, q, s);
  else if (x_dtype == kF16)
    widen ? quant_fp8_group_kernel<kF16, true><<<grid, 256, 0, stream>>>((const uint16_t*)x, rows, cols, ld_x, q, s)
          : quant_fp8_group_kernel<kF16, false><<<grid, 256, 0, stream>>>((const uint16_t*)x, rows, cols, ld_x, q, s);
  else {
    set_last_error("quant_fp8_group: input must be bf16 or fp16");
    return kUnsupported;
  }
  return launch_status("quant_fp8_group");
}

int launch_quant_fp8_row(const void* x, int x_dtype, int64_t rows, int64_t cols, uint8_t* q,
                         float* s, hipStream_t stream) {
  if (rows < 0 || cols <= 0) {
    set_last_error("quant_fp8_row: invalid shape");
    return kInvalidArgument;
  }
  if (rows == 0) return kOk;
  if (x_dtype == kBF16)
    quant_fp8_row_kernel<kBF16><<<(unsigned)rows, 256, 0, stream>>>((const uint16_t*)x, cols, q, s);
  else if (x_dtype == kF16)
    quant_fp8_row_kernel<kF16><<<(unsigned)rows, 256, 0, stream>>>((const uint16_t*)x, cols, q, s);
  else {
    set_last_error("quant_fp8_row: input must be bf16 or fp16");
    return kUnsupported;
  }
  return launch_status("quant_fp8_row");
}

}  // namespace mstar
