// Which lanes of a wave share an LDS cycle in ds_read_b128 (gfx950).
//
// Each launch of lds_probe gives lane l the 16-byte chunk c(l) of its own
// 256-byte row, c(l) = (parity(l & m0), ..., parity(l & m3)) for four lane
// masks: a linear map from the 6 lane-index bits to the 16 bank quads of a
// 256-byte line.  Lanes in different rows that get the same chunk hit the
// same 4 banks.  The kernel repeats the read; with `rocprofv3 --pmc
// SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS` each pattern is one dispatch, and the
// time per read doubles with every two-way conflict.
//
// The model this checks: the 64 lanes are served in four passes of 16, and
// a pass is a coset of the lane subspace spanned by 1, 2, 12 and 24, so lanes
// {0-3, 12-15, 20-23, 24-27} form one pass (and lanes 32-63 likewise).  A map
// is conflict-free exactly when it is one-to-one on that subspace; the
// program prints the model's conflict degree next to the measured time.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <vector>

#define CHECK(x)                                                                         \
  do {                                                                                   \
    hipError_t e_ = (x);                                                                 \
    if (e_ != hipSuccess) {                                                              \
      fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_));           \
      return 1;                                                                          \
    }                                                                                    \
  } while (0)

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kReads = 8, kIters = 2000;

__global__ __launch_bounds__(256) void lds_probe(int m0, int m1, int m2, int m3, int* out) {
  // 16 KB per workgroup of four waves, so 32 waves share a CU's LDS and the
  // reads are throughput-bound, not latency-bound.
  __shared__ __align__(16) uint8_t s[16384];
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < 16384 / 4; i += 256) ((int*)s)[i] = i;
  __syncthreads();
  const int c = (__builtin_popcount(lane & m0) & 1) | ((__builtin_popcount(lane & m1) & 1) << 1) |
                ((__builtin_popcount(lane & m2) & 1) << 2) | ((__builtin_popcount(lane & m3) & 1) << 3);
  v4i acc = {0, 0, 0, 0};
  for (int k = 0; k < kIters; ++k) {
#pragma unroll
    for (int it = 0; it < kReads; ++it)  // row lane ^ it (distinct per lane), chunk c: < 16 KB
      acc += *(const v4i*)(s + (((lane ^ it) & 63) * 16 + c) * 16);
    __asm__ volatile("" ::: "memory");
  }
  out[blockIdx.x * 256 + tid] = acc[0] + acc[1] + acc[2] + acc[3];
}

static int chunk_of(const int m[4], int lane) {
  int c = 0;
  for (int b = 0; b < 4; ++b) c |= (__builtin_popcount(lane & m[b]) & 1) << b;
  return c;
}

// Largest number of lanes of one pass that share a chunk, under the model.
static int model_degree(const int m[4]) {
  const int span[4] = {1, 2, 12, 24};
  std::vector<int> sub = {0};
  for (int v : span) {
    const size_t n = sub.size();
    for (size_t i = 0; i < n; ++i) sub.push_back(sub[i] ^ v);
  }
  int worst = 1;
  bool seen[64] = {};
  for (int b = 0; b < 64; ++b) {
    if (seen[b]) continue;
    int cnt[16] = {};
    for (int s : sub) {
      seen[b ^ s] = true;
      const int k = ++cnt[chunk_of(m, b ^ s)];
      worst = k > worst ? k : worst;
    }
  }
  return worst;
}

int main() {
  // Named patterns, then maps drawn at random (fixed list).
  const int pats[][4] = {
      {1, 2, 4, 8},      // chunk = lane % 16: 16 consecutive lanes distinct
      {1, 2, 4, 16},     // lanes 0-7 and 16-23 distinct
      {1, 2, 16, 32},    // lanes 0-3, 16-19, 32-35, 48-51 distinct
      {1, 2, 4, 32},     // lanes 0-7 and 32-39 distinct
      {1, 2, 4 | 16, 8 | 32},       // l16 ^ 4 lg: the plain XOR swizzle of a 16-row fragment read
      {1, 2, 4 | 16, 8 | 4 | 32},   // the same with bit 3 ^= bit 2: conflict-free under the model
      {40, 17, 48, 23}, {51, 45, 61, 54}, {48, 42, 60, 34}, {2, 54, 30, 50}, {61, 16, 42, 4},
      {58, 11, 8, 24},  {31, 56, 16, 25}, {35, 7, 37, 16},  {1, 47, 14, 27}, {18, 12, 59, 56},
  };
  const int n = sizeof(pats) / sizeof(pats[0]);
  int* d = nullptr;
  const int grid = 2048;  // eight workgroups per CU
  CHECK(hipMalloc(&d, grid * 256 * sizeof(int)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  hipLaunchKernelGGL(lds_probe, dim3(grid), dim3(256), 0, 0, 1, 2, 4, 8, d);  // warm-up
  CHECK(hipDeviceSynchronize());
  printf("masks (m0 m1 m2 m3)        model_degree  ns_per_wave_read_per_CU\n");
  for (int i = 0; i < n; ++i) {
    const int* m = pats[i];
    CHECK(hipEventRecord(e0));
    hipLaunchKernelGGL(lds_probe, dim3(grid), dim3(256), 0, 0, m[0], m[1], m[2], m[3], d);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double per_read = ms * 1e6 / ((double)grid * 4 * kIters * kReads) * 256;  // per CU
    printf("%3d %3d %3d %3d                 %d            %.4f\n", m[0], m[1], m[2], m[3],
           model_degree(m), per_read);
  }
  CHECK(hipFree(d));
  return 0;
}
