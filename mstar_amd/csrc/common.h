// Shared device helpers for the gfx950 fused-MoE kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, the
// OCP e4m3fn FP8 format (not the fnuz variant of gfx942) and the CDNA4
// MFMA instructions v_mfma_f32_16x16x128_f8f6f4 / v_mfma_f32_16x16x32_bf16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mstar {

// ---------------------------------------------------------------- status codes
enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kUnsupported = 2,
  kLaunchError = 3,
  kWorkspaceTooSmall = 4,
};

void set_last_error(const char* fmt, ...);
int launch_status(const char* what);

// ------------------------------------------------------------- element types
enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2, kI32 = 3, kI64 = 4, kFP8 = 5 };

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
constexpr float kFp8Max = 448.0f;
constexpr float kQuantEps = 1e-10f;

// bf16 <-> f32 with round-to-nearest-even, matching torch's float->bfloat16.
// Round to nearest even (NaN stays NaN): the hardware conversion
// (v_cvt_pk_bf16_f32 on gfx950).
__device__ inline uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __host__ inline float bf16_bits_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
__device__ inline float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

__device__ inline uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ inline float f16_bits_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

// 16-bit activation type tag: 1 = bf16, 2 = fp16.
template <int DT>
__device__ inline float h16_to_f32(uint16_t b) {
  if constexpr (DT == kBF16) return bf16_bits_to_f32(b);
  else return f16_bits_to_f32(b);
}
template <int DT>
__device__ inline uint16_t f32_to_h16(float f) {
  if constexpr (DT == kBF16) return f32_to_bf16_bits(f);
  else return f32_to_f16_bits(f);
}
template <int DT>
__device__ inline float round_h16(float f) { return h16_to_f32<DT>(f32_to_h16<DT>(f)); }

// Two floats -> two OCP e4m3fn bytes (RNE, inputs already clamped to +-448),
// packed into the low (hi=false) or high (hi=true) half of `old`.
template <bool HI>
__device__ inline int cvt_pk_fp8(float a, float b, int old) {
  return __builtin_amdgcn_cvt_pk_fp8_f32(a, b, old, HI);
}
// Four floats -> four e4m3fn bytes in one dword (byte i = element i).
__device__ inline int cvt_fp8x4(float a, float b, float c, float d) {
  int v = cvt_pk_fp8<false>(a, b, 0);
  return cvt_pk_fp8<true>(c, d, v);
}
__device__ inline float clamp_fp8(float x) { return fminf(fmaxf(x, -kFp8Max), kFp8Max); }

// ------------------------------------------------------------ wave helpers
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// Max over aligned groups of `W` lanes (W a power of two <= 64).
template <int W>
__device__ inline float group_max(float v) {
#pragma unroll
  for (int o = W / 2; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Eight e4m3fn codes (two dwords) widened exactly to eight bf16 (e4m3fn is a
// subset of bf16).  Whole 32-bit pairs are moved: extracting single __bf16
// elements from the packed results makes the compiler insert byte permutes
// that scramble the pairs.
__device__ __forceinline__ v4i fp8x8_to_bf16x8_bits(int x0, int x1) {
  const int c0 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)x0, 1.0f, false));
  const int c1 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)x0, 1.0f, true));
  const int c2 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)x1, 1.0f, false));
  const int c3 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)x1, 1.0f, true));
  return v4i{c0, c1, c2, c3};
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding: vmcnt low
// bits [3:0], high bits [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without a memory fence (outstanding global loads and LDS
// DMA stay in flight).  The memory clobber keeps the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Workgroup barrier that leaves outstanding global loads in flight: LDS
// traffic is completed (lgkmcnt) but vmcnt is not drained, unlike the
// workgroup fence of __syncthreads().  The memory clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Raw buffer resource over [base, base + bytes): buffer loads at offsets
// >= bytes return zeros without a memory request, which is how lanes with
// nothing to load are masked without a branch.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
constexpr uint32_t kOffNone = 0xFFFFFFF0u;  // an offset no buffer here reaches

// ---- DPP reductions (no LDS round trips).  row_ror:n rotates values
// within each row of 16 lanes; after rotations by 1, 2, 4 and 8 every lane
// of a row holds the row's reduction (association order differs per lane,
// so sums are read from one fixed lane per row).
template <int N>
__device__ __forceinline__ int dpp_row_ror(int v) {
  return __builtin_amdgcn_update_dpp(v, v, 0x120 + N, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t row_umax16(uint32_t v) {
  v = max(v, (uint32_t)dpp_row_ror<1>((int)v));
  v = max(v, (uint32_t)dpp_row_ror<2>((int)v));
  v = max(v, (uint32_t)dpp_row_ror<4>((int)v));
  v = max(v, (uint32_t)dpp_row_ror<8>((int)v));
  return v;
}
__device__ __forceinline__ float row_fmax16(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, dpp_row_ror<1>(__builtin_bit_cast(int, v))));
  v = fmaxf(v, __builtin_bit_cast(float, dpp_row_ror<2>(__builtin_bit_cast(int, v))));
  v = fmaxf(v, __builtin_bit_cast(float, dpp_row_ror<4>(__builtin_bit_cast(int, v))));
  v = fmaxf(v, __builtin_bit_cast(float, dpp_row_ror<8>(__builtin_bit_cast(int, v))));
  return v;
}
__device__ __forceinline__ float row_fsum16(float v) {
  v += __builtin_bit_cast(float, dpp_row_ror<1>(__builtin_bit_cast(int, v)));
  v += __builtin_bit_cast(float, dpp_row_ror<2>(__builtin_bit_cast(int, v)));
  v += __builtin_bit_cast(float, dpp_row_ror<4>(__builtin_bit_cast(int, v)));
  v += __builtin_bit_cast(float, dpp_row_ror<8>(__builtin_bit_cast(int, v)));
  return v;
}
// Wave-uniform results: the four row results combined in row order.
__device__ __forceinline__ uint32_t wave_umax_dpp(uint32_t v) {
  v = row_umax16(v);
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}
__device__ __forceinline__ float wave_fmax_dpp(float v) {
  v = row_fmax16(v);
  const int iv = __builtin_bit_cast(int, v);
  return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16))),
               fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48))));
}
__device__ __forceinline__ float wave_fsum_dpp(float v) {
  v = row_fsum16(v);
  const int iv = __builtin_bit_cast(int, v);
  return ((__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16))) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32))) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
}

// Per-token-group-128 FP8 quantisation of 8 consecutive 16-bit elements
// (raw: 16 bytes of bf16/fp16 bits); the 16 aligned lanes that hold one
// 128-element group cooperate on its amax.  s = max(amax, 1e-10) / 448 and
// q = e4m3fn(clamp(x / s)) with the IEEE quotient and round-to-nearest-even,
// so the codes equal a CPU restatement bit for bit.  Returns the 8 codes.
template <int DT>
__device__ __forceinline__ int2 quant_group8(v4i raw, float& scale) {
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = h16_to_f32<DT>((uint16_t)(raw[i] & 0xffff));
    f[2 * i + 1] = h16_to_f32<DT>((uint16_t)((uint32_t)raw[i] >> 16));
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
  amax = row_fmax16(amax);  // the 16 lanes of a group are one DPP row
  const float sc = fmaxf(amax, kQuantEps) / kFp8Max;
  scale = sc;
  // x / sc as x * (1/sc) plus one FMA residual correction: equal to the IEEE
  // quotient for |x| <= amax (checked over 2M values on the CPU), at a third
  // of the instructions of eight divisions.
  const float rc = 1.0f / sc;
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y0 = f[i] * rc;
    y[i] = clamp_fp8(__builtin_fmaf(__builtin_fmaf(-y0, sc, f[i]), rc, y0));
  }
  return make_int2(cvt_fp8x4(y[0], y[1], y[2], y[3]), cvt_fp8x4(y[4], y[5], y[6], y[7]));
}

// Inclusive prefix sum across the 64 lanes of a wave, by DPP: shifts by
// 1, 2, 4 and 8 lanes within each row of 16, then the last lane of each row
// broadcast into the rows after it (row_bcast:15 into rows 1 and 3,
// row_bcast:31 into rows 2 and 3).  Lanes without a source add 0.
__device__ inline int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// Lane 63's value, wave-uniform (a scalar read, no LDS round trip).
__device__ inline int wave_last(int v) { return __builtin_amdgcn_readlane(v, 63); }

// Eight int4 codes (element j in bits 4j of w, stored as u = q + 8) as the
// bf16 weights bf16((u - 8) * s): the nibbles spread into bytes (even
// elements in lo, odd in hi), each byte converted exactly to fp32
// (v_cvt_f32_ubyteN), fma(u, s, -8 s) (exact: (u - 8) s fits fp32), then
// one rounding of each pair to bf16 (v_cvt_pk_bf16_f32) -- 23 VALU per 8.
// The byte masks are opaque to the compiler, which would otherwise fold
// them into per-nibble bit-field extracts.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v8s int4x8_dequant_bf16(uint32_t w, float s, float m8) {
  uint32_t lo, hi;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(w));
  asm("v_lshrrev_b32 %0, 4, %1\n\tv_and_b32 %0, 0x0f0f0f0f, %0" : "=&v"(hi) : "v"(w));
  v4i r;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const f32x2 e = {__builtin_fmaf((float)((lo >> (8 * b)) & 0xffu), s, m8),
                     __builtin_fmaf((float)((hi >> (8 * b)) & 0xffu), s, m8)};
    r[b] = __builtin_bit_cast(int, __builtin_convertvector(e, bf16x2));
  }
  return __builtin_bit_cast(v8s, r);
}

// Eight int4 codes (element j in bits 4j of w) as bf16 128 + u, two per
// dword in the order 0, 4, 1, 5, 2, 6, 3, 7: 128 + u is bf16 0x4300 | u.  A
// dot product over these values is sum (u + 128) x; sum (u - 8) x follows
// by subtracting 136 sum x.  Each pair is one v_bfi_b32 (mask m =
// 0x000f000f in an SGPR, bias c = 0x43004300 in a VGPR: both from
// int4_bias_consts) after a shift.
struct Int4BiasConsts {
  uint32_t m, c;
};
__device__ __forceinline__ Int4BiasConsts int4_bias_consts() {
  Int4BiasConsts k;
  asm volatile("s_mov_b32 %0, 0x000f000f" : "=s"(k.m));
  asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(k.c));
  return k;
}
// The bit-field insert is written in C (the compiler selects v_bfi_b32 and,
// unlike for inline assembly, inserts the wait states an MFMA reading its
// result needs); the constants are opaque so that it is not folded into an
// and and an or.
__device__ __forceinline__ v8s int4x8_bias128(uint32_t w, Int4BiasConsts k) {
  v4i r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = (int)(((w >> (4 * j)) & k.m) | (k.c & ~k.m));
  return __builtin_bit_cast(v8s, r);
}

// ---------------------------------------------------------------- MFMA
// 16x16x128 FP8 (e4m3fn x e4m3fn), fp32 accumulate.  Operand layout (both A
// and B): lane l supplies row/column (l % 16) and 32 consecutive K bytes at
// K offset (l / 16) * 32.  Result: lane l holds C[4*(l/16) + r][l % 16].
__device__ inline v4f mfma_fp8_16x16x128(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// 32x32x64 FP8: lane l supplies row/column (l % 32) and 32 consecutive K
// bytes at K offset (l / 32) * 32.  Result: lane l, register i holds
// C[8*(i/4) + 4*(l/32) + (i%4)][l % 32].
typedef float v16f __attribute__((ext_vector_type(16)));
__device__ inline v16f mfma_fp8_32x32x64(v8i a, v8i b, v16f c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// 16x16x32 bf16 / fp16: lane l supplies row (l % 16) and 8 consecutive K
// elements at K offset (l / 16) * 8.  Same C layout as above.
__device__ inline v4f mfma_bf16_16x16x32(v8s a, v8s b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a),
                                                 __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
}
__device__ inline v4f mfma_f16_16x16x32(v8s a, v8s b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a),
                                                __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}
template <int DT>
__device__ inline v4f mfma_h16(v8s a, v8s b, v4f c) {
  if constexpr (DT == kBF16) return mfma_bf16_16x16x32(a, b, c);
  else return mfma_f16_16x16x32(a, b, c);
}

// One routing weight, stored as fp32, bf16 or fp16.
__device__ inline float load_weight_any(const void* w, int dtype, int64_t i) {
  if (dtype == kF32) return ((const float*)w)[i];
  const uint16_t b = ((const uint16_t*)w)[i];
  return dtype == kBF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// x * sigmoid(x) with the hardware reciprocal (about 1 ulp); the callers
// round the result to bf16.
__device__ inline float silu_f32(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ inline float gelu_tanh_f32(float x) {
  const float k = 0.7978845608028654f;
  float t = k * (x + 0.044715f * x * x * x);
  float th = 2.0f * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * t)) - 1.0f;
  return 0.5f * x * (1.0f + th);
}
template <int ACT>
__device__ inline float act_f32(float x) {
  if constexpr (ACT == 0) return silu_f32(x);
  else return gelu_tanh_f32(x);
}

}  // namespace mstar
