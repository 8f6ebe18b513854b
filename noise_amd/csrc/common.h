// Shared definitions of the noise_amd HIP library (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/noise_amd.h"

typedef uint16_t bf16_t;  // storage type of bfloat16 in global memory
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

// The fixed model's widths (utils/model.py:34-43, 69-79, 100-104).
constexpr int kD = 512;       // n_embd
constexpr int kH = 8;         // heads
constexpr int kHD = 64;       // head_dim
constexpr int kF = 2048;      // MLP hidden
constexpr int kGateIn = 32;   // ve_gate input channels
constexpr int kQKV = 3 * kD;  // fused q|k|v output width

__device__ __forceinline__ float bf16_to_f32(bf16_t v) { return __uint_as_float(((uint32_t)v) << 16); }

// Round-to-nearest-even fp32 -> bf16, the rounding of torch's .to(torch.bfloat16) (gfx950 converts in hardware).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// Two floats as a bf16 pair (low half first), and back. The pair converts as a 2-vector, one v_cvt_pk_bf16_f32
// (round to nearest even per element, as f32_to_bf16) instead of two conversions, a shift and an or.
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_v{lo, hi}), bf16x2_v));
}
__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }
// c + a.lo b.lo + a.hi b.hi over bf16 pairs (v_dot2_f32_bf16: exact bf16 products, fp32 sum)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a), __builtin_bit_cast(bf16x2_v, b), c, false);
}

typedef short v4s __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
// gfx950 transposing LDS read (ds_read_b64_tr_b16), spelled out in the device pass only.
__device__ __forceinline__ v4s ds_read_tr16(const bf16_t* p) {
#if __HIP_DEVICE_COMPILE__
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(__attribute__((address_space(3))) void*)(void*)p);
#else
  (void)p;
  return v4s{0, 0, 0, 0};
#endif
}

// Hardware 2^x and 1/x (v_exp_f32, v_rcp_f32: about 1 ulp, no denormal-range fix-ups), for softmax weights and
// soft caps whose arguments are bounded.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
// 1/sqrt(x) for x >= the RMS-norm epsilon: v_rsq_f32 alone. rsqrtf adds a rescaling that changes only denormal
// inputs, which these arguments (a mean square plus eps = 2^-23) never are.
__device__ __forceinline__ float rsq_norm(float x) { return __builtin_amdgcn_rsqf(x); }


// Cross-lane moves without the LDS crossbar. dpp_mov<CTRL>: a DPP row control (0xB1 quad_perm [1,0,3,2], 0x4E
// quad_perm [2,3,0,1], 0x141 row_half_mirror, 0x140 row_mirror, 0x128 row_ror:8). lane_swap32(a, b): a takes
// {a[0:31], b[0:31]} and b takes {a[32:63], b[32:63]} (v_permlane32_swap). lane_swap16(a, b): rows of 16 lanes,
// a takes {a.r0, b.r0, a.r2, b.r2} and b takes {a.r1, b.r1, a.r3, b.r3} (v_permlane16_swap). The builtins are
// spelled out in the device pass only.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
#if __HIP_DEVICE_COMPILE__
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
#else
  return x;
#endif
}
__device__ __forceinline__ void lane_swap32(float& a, float& b) {
#if __HIP_DEVICE_COMPILE__
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
#endif
}
__device__ __forceinline__ void lane_swap16(float& a, float& b) {
#if __HIP_DEVICE_COMPILE__
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
#endif
}
// x of lane l ^ 32.
__device__ __forceinline__ float lane_xor32(float x, int lane) {
  float a = x, b = x;
  lane_swap32(a, b);  // a: {x[0:31], x[0:31]}, b: {x[32:63], x[32:63]}
  return (lane & 32) ? a : b;
}
// Sum over each 8-lane group, in every lane of the group (each step adds a lane's partner, so all lanes agree).
__device__ __forceinline__ float group_sum8(float c) {
  c += dpp_mov<0xB1>(c);
  c += dpp_mov<0x4E>(c);
  c += dpp_mov<0x141>(c);
  return c;
}

// Sums of 4 per-lane values over the 64 lanes, by a transposed butterfly (halves swapped, then rows, then within a
// row): returns the total of value (2 b5 + b4), b5 b4 = bits 5..4 of the lane id (the 16 lanes of row q hold the
// total of value q).
__device__ __forceinline__ float warp_sum4(const float (&p)[4], int) {
  float a0 = p[0], b0 = p[2], a1 = p[1], b1 = p[3];
  lane_swap32(a0, b0);
  lane_swap32(a1, b1);
  float s0 = a0 + b0, s1 = a1 + b1;  // lanes 0..31: values 0, 1; lanes 32..63: values 2, 3
  lane_swap16(s0, s1);
  const float c = group_sum8(s0 + s1);
  return c + dpp_mov<0x140>(c);
}

// x as held by lane idx; idx must be the same in every lane (v_readlane_b32).
__device__ __forceinline__ float lane_val(float x, int idx) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), idx));
}
__device__ __forceinline__ int lane_val(int x, int idx) { return __builtin_amdgcn_readlane(x, idx); }

// Sums of 8 per-lane values over the 64 lanes, by a transposed butterfly (halves, rows, half-rows, then within 8
// lanes): returns the total of value (4 b5 + 2 b4 + b3) where b5 b4 b3 are bits 5..3 of the lane id (8 lanes hold
// each total).
__device__ __forceinline__ float warp_sum8(const float (&p)[8], int lane) {
  float q[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float a = p[r], b = p[r + 4];
    lane_swap32(a, b);
    q[r] = a + b;  // lanes 0..31: value r; lanes 32..63: value r + 4
  }
  float w[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    float a = q[r], b = q[r + 2];
    lane_swap16(a, b);
    w[r] = a + b;  // rows 0..3: values r, r + 2, r + 4, r + 6
  }
  const bool b3 = lane & 8;
  const float z = (b3 ? w[1] : w[0]) + dpp_mov<0x128>(b3 ? w[0] : w[1]);
  return group_sum8(z);
}

// Sum / max over the 64 lanes, in every lane (halves, rows, then within a row; each step combines a lane with its
// partner, so all lanes agree).
__device__ __forceinline__ float warp_sum(float v) {
  const int lane = __lane_id();
  {
    float a = v, b = v;
    lane_swap32(a, b);
    v += (lane & 32) ? a : b;
  }
  {
    float a = v, b = v;
    lane_swap16(a, b);  // a: {r0, r0, r2, r2}, b: {r1, r1, r3, r3}
    v += (lane & 16) ? a : b;
  }
  v = group_sum8(v);
  return v + dpp_mov<0x140>(v);
}
__device__ __forceinline__ float warp_max(float v) {
  const int lane = __lane_id();
  {
    float a = v, b = v;
    lane_swap32(a, b);
    v = fmaxf(v, (lane & 32) ? a : b);
  }
  {
    float a = v, b = v;
    lane_swap16(a, b);
    v = fmaxf(v, (lane & 16) ? a : b);
  }
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  return fmaxf(v, dpp_mov<0x140>(v));
}

// Error state of the C ABI (abi.cpp).
int noise_set_error(int code, const char* fmt, ...);

#define NOISE_CHECK_HIP(expr)                                                                   \
  do {                                                                                          \
    hipError_t _e = (expr);                                                                     \
    if (_e != hipSuccess)                                                                       \
      return noise_set_error(NOISE_ERR_HIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), \
                             __FILE__, __LINE__);                                               \
  } while (0)

#define NOISE_REQUIRE(cond, ...)                                   \
  do {                                                             \
    if (!(cond)) return noise_set_error(NOISE_ERR_ARG, __VA_ARGS__); \
  } while (0)

#define NOISE_LAUNCH_CHECK() NOISE_CHECK_HIP(hipGetLastError())

// Per-kernel-class launch timing (diagnostics, off by default): when enabled, launches are bracketed by hipEvent
// pairs recorded on their stream; noise_timing_read() reports counts and summed durations per class.
enum NoiseTimingClass {
  kTimeNoise = 0, kTimeEmbed, kTimeNorm, kTimeQKV, kTimeRope, kTimeAttention, kTimeProj, kTimeFc, kTimeRowdot,
  kTimeMlpProj, kTimeHead, kTimeCeFinal, kTimeCreditLse, kTimeCreditValue, kTimeUpdate, kTimeLowrank, kTimeCreditCenter, kTimeHeadError, kTimeDustRerun, kTimeDustErrors,
  kTimeLowrankPre, kTimeLowrankPost, kTimeFitness, kTimeVectorGrad, kTimeAdamw, kTimeReassemble, kTimeLinear,
  kTimeClasses
};

struct NoiseTimer {
  int slot;
  hipStream_t stream;
  NoiseTimer(int cls, hipStream_t s);
  ~NoiseTimer();
};
