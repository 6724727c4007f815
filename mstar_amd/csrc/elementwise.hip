// Activation-and-multiply and the top-k sum-reduce.
//
//  * act_and_mul_kernel restates act_and_mul_kernel
//    (mstar/utils/fused_moe/kernels.py:244-276): out = dt(dt(act_f32(gate)) * up)
//    with gate = columns [0, I), up = columns [I, 2I).
//  * sum_reduce_kernel restates moe_sum_reduce_kernel (kernels.py:306-356):
//    fp32 sum over the top-k dimension, times the scaling factor, cast.
// Both move 16 bytes per lane per access; sizes that are not a multiple of
// 8 elements take one-element-per-thread variants.
#include "common.h"
#include "launch.h"

namespace mstar {

template <int DT, int ACT>
__global__ __launch_bounds__(256) void act_and_mul_kernel(const uint16_t* __restrict__ gu,
                                                          uint16_t* __restrict__ out,
                                                          int64_t rows, int64_t inter) {
  const int64_t vecs_per_row = inter / 8;
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= rows * vecs_per_row) return;
  const int64_t r = v / vecs_per_row, c = (v % vecs_per_row) * 8;
  v4i g = *(const v4i*)(gu + r * 2 * inter + c);
  v4i u = *(const v4i*)(gu + r * 2 * inter + inter + c);
  v4i o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t gw = (uint32_t)g[i], uw = (uint32_t)u[i];
    float g0 = h16_to_f32<DT>(gw & 0xffff), g1 = h16_to_f32<DT>(gw >> 16);
    float u0 = h16_to_f32<DT>(uw & 0xffff), u1 = h16_to_f32<DT>(uw >> 16);
    float a0 = round_h16<DT>(act_f32<ACT>(g0)), a1 = round_h16<DT>(act_f32<ACT>(g1));
    o[i] = (int)((uint32_t)f32_to_h16<DT>(a0 * u0) | ((uint32_t)f32_to_h16<DT>(a1 * u1) << 16));
  }
  *(v4i*)(out + r * inter + c) = o;
}

// POS: row j of token t is in[pos_of[t * topk + j]] (rows by sorted
// position) instead of in[t * topk + j].
template <int DT, bool POS>
__global__ __launch_bounds__(256) void sum_reduce_kernel(const uint16_t* __restrict__ in,
                                                         const int32_t* __restrict__ pos_of,
                                                         uint16_t* __restrict__ out,
                                                         int64_t tokens, int topk,
                                                         int64_t hidden, float scale) {
  const int64_t vecs = hidden / 8;
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= tokens * vecs) return;
  const int64_t t = v / vecs, c = (v % vecs) * 8;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto add = [&](const v4i& x) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += h16_to_f32<DT>((uint32_t)x[i] & 0xffff);
      acc[2 * i + 1] += h16_to_f32<DT>((uint32_t)x[i] >> 16);
    }
  };
  // Eight rows at a time: their loads (and, by position, the position loads
  // before them) are all in flight together; the sum stays in row order.
  int j = 0;
  for (; j + 8 <= topk; j += 8) {
    int64_t row[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) row[u] = POS ? (int64_t)pos_of[t * topk + j + u] : t * topk + j + u;
    v4i x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      // By position (the 256-row prefill GEMM's output, stored non-temporally
      // and read once): non-temporal loads too.
      const v4i* src = (const v4i*)(in + row[u] * hidden + c);
      x[u] = POS ? __builtin_nontemporal_load(src) : *src;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) add(x[u]);
  }
  for (; j < topk; ++j) {
    const int64_t row = POS ? (int64_t)pos_of[t * topk + j] : t * topk + j;
    add(*(const v4i*)(in + row * hidden + c));
  }
  v4i o;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = (int)((uint32_t)f32_to_h16<DT>(acc[2 * i] * scale) |
                 ((uint32_t)f32_to_h16<DT>(acc[2 * i + 1] * scale) << 16));
  *(v4i*)(out + t * hidden + c) = o;
}

// One element per thread: sizes that are not a multiple of 8 elements, or
// rows not 16-byte aligned.  Same arithmetic as the vector kernels.
template <int DT, int ACT>
__global__ __launch_bounds__(256) void act_and_mul_scalar_kernel(const uint16_t* __restrict__ gu,
                                                                 uint16_t* __restrict__ out,
                                                                 int64_t rows, int64_t inter) {
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= rows * inter) return;
  const int64_t r = v / inter, c = v % inter;
  const float g = h16_to_f32<DT>(gu[r * 2 * inter + c]);
  const float u = h16_to_f32<DT>(gu[r * 2 * inter + inter + c]);
  out[v] = f32_to_h16<DT>(round_h16<DT>(act_f32<ACT>(g)) * u);
}

template <int DT>
__global__ __launch_bounds__(256) void sum_reduce_scalar_kernel(const uint16_t* __restrict__ in,
                                                                uint16_t* __restrict__ out,
                                                                int64_t tokens, int topk,
                                                                int64_t hidden, float scale) {
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= tokens * hidden) return;
  const int64_t t = v / hidden, c = v % hidden;
  float acc = 0.f;
  for (int j = 0; j < topk; ++j) acc += h16_to_f32<DT>(in[(t * topk + j) * hidden + c]);
  out[v] = f32_to_h16<DT>(acc * scale);
}

static bool aligned16(const void* a, const void* b) {
  return (((uintptr_t)a | (uintptr_t)b) & 15) == 0;
}

int launch_act_and_mul(const void* gate_up, void* out, int dtype, int64_t rows, int64_t inter,
                       int activation, hipStream_t stream) {
  if (rows < 0 || inter <= 0 || (activation != 0 && activation != 1)) {
    set_last_error("act_and_mul: inter must be positive and activation 0 or 1 (inter=%lld)",
                   (long long)inter);
    return kInvalidArgument;
  }
  if (rows == 0) return kOk;
  if (inter % 8 != 0 || !aligned16(gate_up, out)) {
    dim3 g1((unsigned)((rows * inter + 255) / 256));
    const uint16_t* gu = (const uint16_t*)gate_up;
    uint16_t* o = (uint16_t*)out;
    if (dtype == kBF16 && activation == 0) act_and_mul_scalar_kernel<kBF16, 0><<<g1, 256, 0, stream>>>(gu, o, rows, inter);
    else if (dtype == kBF16) act_and_mul_scalar_kernel<kBF16, 1><<<g1, 256, 0, stream>>>(gu, o, rows, inter);
    else if (dtype == kF16 && activation == 0) act_and_mul_scalar_kernel<kF16, 0><<<g1, 256, 0, stream>>>(gu, o, rows, inter);
    else if (dtype == kF16) act_and_mul_scalar_kernel<kF16, 1><<<g1, 256, 0, stream>>>(gu, o, rows, inter);
    else {
      set_last_error("act_and_mul: dtype must be bf16 or fp16");
      return kUnsupported;
    }
    return launch_status("act_and_mul");
  }
  dim3 grid((unsigned)((rows * (inter / 8) + 255) / 256));
  const uint16_t* gu = (const uint16_t*)gate_up;
  uint16_t* o = (uint16_t*)out;
  if (dtype == kBF16 && activation == 0) act_and_mul_kernel<kBF16, 0><<<grid, 256, 0, stream>>>(gu, o, rows, inter);
  else if (dtype == kBF16) act_and_mul_kernel<kBF16, 1><<<grid, 256, 0, stream>>>(gu, o, rows, inter);
  else if (dtype == kF16 && activation == 0) act_and_mul_kernel<kF16, 0><<<grid, 256, 0, stream>>>(gu, o, rows, inter);
  else if (dtype == kF16) act_and_mul_kernel<kF16, 1><<<grid, 256, 0, stream>>>(gu, o, rows, inter);
  else {
    set_last_error("act_and_mul: dtype must be bf16 or fp16");
    return kUnsupported;
  }
  return launch_status("act_and_mul");
}

int launch_sum_reduce(const void* in, void* out, int dtype, int64_t tokens, int64_t topk,
                      int64_t hidden, float scale, hipStream_t stream) {
  if (tokens < 0 || topk <= 0 || topk > INT32_MAX || hidden <= 0) {
    set_last_error("moe_sum_reduce: invalid sizes (tokens=%lld top_k=%lld hidden=%lld)",
                   (long long)tokens, (long long)topk, (long long)hidden);
    return kInvalidArgument;
  }
  if (tokens == 0) return kOk;
  if (hidden % 8 != 0 || !aligned16(in, out)) {
    dim3 g1((unsigned)((tokens * hidden + 255) / 256));
    if (dtype == kBF16)
      sum_reduce_scalar_kernel<kBF16><<<g1, 256, 0, stream>>>((const uint16_t*)in, (uint16_t*)out, tokens,
                                                               (int)topk, hidden, scale);
    else if (dtype == kF16)
      sum_reduce_scalar_kernel<kF16><<<g1, 256, 0, stream>>>((const uint16_t*)in, (uint16_t*)out, tokens,
                                                              (int)topk, hidden, scale);
    else {
      set_last_error("moe_sum_reduce: dtype must be bf16 or fp16");
      return kUnsupported;
    }
    return launch_status("moe_sum_reduce");
  }
  dim3 grid((unsigned)((tokens * (hidden / 8) + 255) / 256));
  if (dtype == kBF16)
    sum_reduce_kernel<kBF16, false><<<grid, 256, 0, stream>>>((const uint16_t*)in, nullptr, (uint16_t*)out, tokens,
                                                       (int)topk, hidden, scale);
  else if (dtype == kF16)
    sum_reduce_kernel<kF16, false><<<grid, 256, 0, stream>>>((const uint16_t*)in, nullptr, (uint16_t*)out, tokens,
                                                      (int)topk, hidden, scale);
  else {
    set_last_error("moe_sum_reduce: dtype must be bf16 or fp16");
    return kUnsupported;
  }
  return launch_status("moe_sum_reduce");
}

int launch_sum_reduce_pos(const void* in, const int32_t* pos_of, void* out, int dtype,
                          int64_t tokens, int64_t topk, int64_t hidden, hipStream_t stream) {
  if (tokens < 0 || topk <= 0 || hidden <= 0 || hidden % 8 != 0 || (tokens > 0 && !pos_of)) {
    set_last_error("moe_sum_reduce: hidden must be a positive multiple of 8 (hidden=%lld)",
                   (long long)hidden);
    return kInvalidArgument;
  }
  if (tokens == 0) return kOk;
  dim3 grid((unsigned)((tokens * (hidden / 8) + 255) / 256));
  if (dtype == kBF16)
    sum_reduce_kernel<kBF16, true><<<grid, 256, 0, stream>>>((const uint16_t*)in, pos_of, (uint16_t*)out,
                                                             tokens, (int)topk, hidden, 1.0f);
  else if (dtype == kF16)
    sum_reduce_kernel<kF16, true><<<grid, 256, 0, stream>>>((const uint16_t*)in, pos_of, (uint16_t*)out,
                                                            tokens, (int)topk, hidden, 1.0f);
  else {
    set_last_error("moe_sum_reduce: dtype must be bf16 or fp16");
    return kUnsupported;
  }
  return launch_status("moe_sum_reduce");
}

}  // namespace mstar
