// Machine ceilings the kernels' rooflines are quoted against, measured on
// the device this runs on:
//   hbm_read   -- streaming read of a 2 GiB buffer (16-byte non-temporal
//                 loads, grid-stride over every CU): achievable HBM read rate;
//   hbm_read_lds -- the same read through LDS-DMA (global_load_lds, 16 bytes a
//                 lane, non-temporal), each wave keeping 16 KB in flight, the
//                 way the decode weight-streaming kernels read;
//   hbm_copy   -- 1 GiB read + 1 GiB written: the copy rate;
//   mfma_fp8   -- v_mfma_f32_32x32x64_f8f6f4, eight independent accumulator
//                 chains per wave, four waves per SIMD: dense FP8 MFMA rate;
//   mfma_bf16  -- v_mfma_f32_32x32x16_bf16, the same shape of loop;
//   fp8_precision -- one 32x32x64 FP8 MFMA against the exact (float64) sum
//                 of its 64 products: how far its internal accumulation is
//                 from fp32.
// Output: one line per measurement.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <vector>

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) void hbm_read(const v4i* __restrict__ p, int64_t n, int* out) {
  v4i acc = {0, 0, 0, 0};
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    v4i a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
    v4i c = __builtin_nontemporal_load(p + i + 2 * stride), d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n; i += stride) acc ^= __builtin_nontemporal_load(p + i);
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x7e1f2d3c) out[0] = 1;  // keeps the loads
}

typedef __attribute__((address_space(3))) void* lds_void_ptr;
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Each wave streams 1 KB pieces (64 lanes x 16 B) of consecutive 16 KB
// blocks into its own 16-slot LDS ring, waiting only for the piece 16
// issues back.  Nothing reads the LDS: this is the DMA's rate alone.
__global__ __launch_bounds__(256) void hbm_read_lds(const uint8_t* __restrict__ p, int64_t blocks) {
  __shared__ __align__(16) uint8_t ring[4][16][1024];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t nw = (int64_t)gridDim.x * 4;
  for (int64_t b = (int64_t)blockIdx.x * 4 + w; b < blocks; b += nw) {
    const uint8_t* src = p + b * 16384 + lane * 16;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      __builtin_amdgcn_global_load_lds((const void*)(src + s * 1024), (lds_void_ptr)&ring[w][s][0], 16, 0, 2);
      wait_vmcnt<15>();
    }
  }
  wait_vmcnt<0>();
}

__global__ __launch_bounds__(256) void hbm_copy(const v4i* __restrict__ p, v4i* __restrict__ q, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(p + i), q + i);
}

template <bool FP8>
__global__ __launch_bounds__(256) void mfma_loop(int iters, float* out) {
  v8i a8 = {(int)threadIdx.x, 1, 2, 3, 4, 5, 6, 7};
  v8s a16 = {(short)threadIdx.x, 1, 2, 3, 4, 5, 6, 7};
  v16f acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = v16f{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if constexpr (FP8)
        acc[c] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, a8, acc[c], 0, 0, 0, 0, 0, 0);
      else
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a16),
                                                         __builtin_bit_cast(v8bf, a16), acc[c], 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[c][e];
  if (s == 1234.5f) out[0] = s;
}

__global__ void fp8_dot(const uint8_t* A, const uint8_t* B, float* C) {
  const int w = blockIdx.x, l = threadIdx.x;
  const uint8_t* a = A + (size_t)w * 2048;
  const uint8_t* b = B + (size_t)w * 2048;
  v8i av = *(const v8i*)(a + (l % 32) * 64 + (l / 32) * 32);
  v8i bv = *(const v8i*)(b + (l % 32) * 64 + (l / 32) * 32);
  v16f c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, v16f{}, 0, 0, 0, 0, 0, 0);
  for (int i = 0; i < 16; ++i) C[(size_t)w * 1024 + (8 * (i / 4) + 4 * (l / 32) + (i % 4)) * 32 + l % 32] = c[i];
}

static double e4m3(uint8_t v) {
  const int e = (v >> 3) & 15, m = v & 7;
  const double r = e == 0 ? ldexp(m / 8.0, -6) : ldexp(1 + m / 8.0, e - 7);
  return (v >> 7) ? -r : r;
}

template <typename F>
static double median_ms(F launch, int reps) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  launch();  // warm-up
  std::vector<float> t;
  for (int r = 0; r < reps; ++r) {
    CHECK(hipEventRecord(a));
    launch();
    CHECK(hipEventRecord(b));
    CHECK(hipEventSynchronize(b));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, a, b));
    t.push_back(ms);
  }
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

int main() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  int* flag;
  CHECK(hipMalloc(&flag, 4));
  {
    const int64_t bytes = (int64_t)2 << 30, n = bytes / 16;
    v4i* p;
    CHECK(hipMalloc(&p, bytes));
    CHECK(hipMemset(p, 1, bytes));
    const double ms = median_ms([&] { hbm_read<<<cus * 8, 256>>>(p, n, flag); }, 20);
    printf("hbm_read: %.0f GB/s (2 GiB, median of 20)\n", bytes / ms / 1e6);
    const double msl = median_ms([&] { hbm_read_lds<<<cus * 2, 256>>>((const uint8_t*)p, bytes / 16384); }, 20);
    printf("hbm_read_lds: %.0f GB/s (2 GiB through LDS-DMA, 8 waves per CU, median of 20)\n",
           bytes / msl / 1e6);
    const int64_t half = bytes / 2;
    const double ms2 = median_ms([&] { hbm_copy<<<cus * 8, 256>>>(p, p + half / 16, half / 16); }, 20);
    printf("hbm_copy: %.0f GB/s read+write (1 GiB each way, median of 20)\n", 2.0 * half / ms2 / 1e6);
    CHECK(hipFree(p));
  }
  {
    float* out;
    CHECK(hipMalloc(&out, 4));
    const int iters = 2000, blocks = cus * 4;  // 16 waves per CU, 4 per SIMD
    const double waves = blocks * 4.0;
    double ms = median_ms([&] { mfma_loop<true><<<blocks, 256>>>(iters, out); }, 10);
    printf("mfma_fp8: %.0f TFLOP/s (32x32x64 f8f6f4, %d CUs)\n",
           waves * iters * 8 * 2.0 * 32 * 32 * 64 / ms / 1e9, cus);
    ms = median_ms([&] { mfma_loop<false><<<blocks, 256>>>(iters, out); }, 10);
    printf("mfma_bf16: %.0f TFLOP/s (32x32x16 bf16)\n", waves * iters * 8 * 2.0 * 32 * 32 * 16 / ms / 1e9);
    CHECK(hipFree(out));
  }
  {
    const int W = 2048;
    const size_t n = (size_t)W * 2048;
    std::vector<uint8_t> hA(n), hB(n);
    srand(1);
    auto code = [] {  // finite e4m3 codes with exponent field 2..14
      uint8_t v;
      do v = (uint8_t)(rand() & 0xff); while (((v >> 3) & 15) == 15 || ((v >> 3) & 15) < 2);
      return v;
    };
    for (size_t i = 0; i < n; ++i) { hA[i] = code(); hB[i] = code(); }
    uint8_t *dA, *dB;
    float* dC;
    CHECK(hipMalloc(&dA, n));
    CHECK(hipMalloc(&dB, n));
    CHECK(hipMalloc(&dC, (size_t)W * 1024 * 4));
    CHECK(hipMemcpy(dA, hA.data(), n, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dB, hB.data(), n, hipMemcpyHostToDevice));
    fp8_dot<<<W, 64>>>(dA, dB, dC);
    std::vector<float> hC((size_t)W * 1024);
    CHECK(hipMemcpy(hC.data(), dC, hC.size() * 4, hipMemcpyDeviceToHost));
    double se = 0, sv = 0, smax = 0, rel_max = 0;
    long differ = 0, cnt = 0;
    for (int w = 0; w < W; ++w)
      for (int r = 0; r < 32; ++r)
        for (int c = 0; c < 32; ++c) {
          double ex = 0, mag = 0;
          for (int k = 0; k < 64; ++k) {
            const double p = e4m3(hA[(size_t)w * 2048 + r * 64 + k]) * e4m3(hB[(size_t)w * 2048 + c * 64 + k]);
            ex += p;
            mag = fmax(mag, fabs(p));
          }
          const double err = hC[(size_t)w * 1024 + r * 32 + c] - ex;
          se += err * err;
          sv += ex * ex;
          smax += fabs(err) / mag;
          rel_max = fmax(rel_max, fabs(err) / mag);
          differ += (float)ex != hC[(size_t)w * 1024 + r * 32 + c];
          ++cnt;
        }
    printf("fp8_precision: rms(err)/rms(sum) %.2e, mean |err|/max|product| %.2e, max %.2e; "
           "%.2f%% of outputs differ from the fp32-rounded exact sum (%ld dots of 64)\n",
           sqrt(se / sv), smax / cnt, rel_max, 100.0 * differ / cnt, cnt);
  }
  return 0;
}
