// Counter-based perturbation noise on the device: Philox4x32-10 (Salmon et al., SC'11) and Box-Muller through
// this library's own polynomial ln / sin / cos. Every float operation is written out (explicit fmaf, contraction
// off) so the values equal, bit for bit, those of the CPU restatement in the test suite's oracle.
//
//   G[i] (i < 2^28)     = lane (i & 3) of BoxMuller2(philox((i >> 2, 0, 0, kStreamBuffer), (seed_lo, seed_hi)))
//   off_p[d] at step s  = (philox((d, p, 0, kStreamOffset), lo/hi(1000003 * seed + s))[0] * range) >> 32
//
// Replaces the reference's fixed torch.randn buffer and torch.randint offsets
// (archive/10M/train/val/eggroll.py:35, 114, 117-128), keeping its slicing algebra.
#pragma once

#include "common.h"

namespace noise {

constexpr uint32_t kStreamBuffer = 0x4E4F4953u;
constexpr uint32_t kStreamOffset = 0x4F464653u;
constexpr uint32_t kStreamHead = 0x44414548u;  // the head-slab estimator's per-draw logit jitter
constexpr uint32_t kStreamDust = 0x54535544u;  // the direct draws' per-draw activation jitter
constexpr uint64_t kNoiseSize = 1ull << 28;

struct u32x4s { uint32_t x, y, z, w; };

__device__ __forceinline__ u32x4s philox4x32_10(u32x4s c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = 0xD2511F53u * c.x, hi0 = __umulhi(0xD2511F53u, c.x);
    const uint32_t lo1 = 0xCD9E8D57u * c.z, hi1 = __umulhi(0xCD9E8D57u, c.z);
    c = u32x4s{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

// ln(u), u in (0, 1]: u = m 2^e, m in (sqrt(1/2), sqrt(2)], ln m = 2 s (1 + s^2/3 + ... + s^10/11), s = (m-1)/(m+1).
__device__ __forceinline__ float ln_unit(float u) {
#pragma clang fp contract(off)
  uint32_t bits = __float_as_uint(u);
  int e = (int)((bits >> 23) & 0xFF) - 127;
  float m = __uint_as_float((bits & 0x007FFFFFu) | 0x3F800000u);
  if (m > 1.41421356f) { m = m * 0.5f; e = e + 1; }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float z = s * s;
  float p = 1.0f / 11.0f;
  p = __builtin_fmaf(p, z, 1.0f / 9.0f);
  p = __builtin_fmaf(p, z, 1.0f / 7.0f);
  p = __builtin_fmaf(p, z, 1.0f / 5.0f);
  p = __builtin_fmaf(p, z, 1.0f / 3.0f);
  p = __builtin_fmaf(p, z, 1.0f);
  const float lnm = 2.0f * s * p;
  const float fe = (float)e;
  return __builtin_fmaf(fe, 0.693145751953125f, __builtin_fmaf(fe, 1.42860682030941723212e-6f, lnm));
}

// (sin, cos) of 2 pi u for u = k 2^-24 in [0, 1): exact quadrant split 4u = q + f, angle q pi/2 + pi/4 + phi,
// phi = (f - 1/2) pi/2, Taylor polynomials through phi^9 / phi^10.
__device__ __forceinline__ void sincos_2pi(float u, float* sn, float* cs) {
#pragma clang fp contract(off)
  const float t = u * 4.0f;
  const int q = (int)t;
  const float f = t - (float)q;
  const float phi = (f - 0.5f) * 1.57079632679489662f;
  const float z = phi * phi;
  float ps = 1.0f / 362880.0f;
  ps = __builtin_fmaf(ps, z, -1.0f / 5040.0f);
  ps = __builtin_fmaf(ps, z, 1.0f / 120.0f);
  ps = __builtin_fmaf(ps, z, -1.0f / 6.0f);
  ps = __builtin_fmaf(ps, z, 1.0f);
  const float s = phi * ps;
  float pc = -1.0f / 3628800.0f;
  pc = __builtin_fmaf(pc, z, 1.0f / 40320.0f);
  pc = __builtin_fmaf(pc, z, -1.0f / 720.0f);
  pc = __builtin_fmaf(pc, z, 1.0f / 24.0f);
  pc = __builtin_fmaf(pc, z, -0.5f);
  const float c = __builtin_fmaf(pc, z, 1.0f);
  const float r = 0.70710678118654752f;
  const float c45 = (c - s) * r, s45 = (c + s) * r;
  if (q == 0) { *cs = c45; *sn = s45; }
  else if (q == 1) { *cs = -s45; *sn = c45; }
  else if (q == 2) { *cs = -c45; *sn = -s45; }
  else { *cs = s45; *sn = -c45; }
}

__device__ __forceinline__ void box_muller(uint32_t x, uint32_t y, float* z0, float* z1) {
#pragma clang fp contract(off)
  const float u1 = (float)((x >> 8) + 1u) * 5.9604644775390625e-8f;
  const float u2 = (float)(y >> 8) * 5.9604644775390625e-8f;
  const float r = __builtin_sqrtf(-2.0f * ln_unit(u1));
  float sn, cs;
  sincos_2pi(u2, &sn, &cs);
  *z0 = r * cs;
  *z1 = r * sn;
}

// The four buffer values G[4 blk .. 4 blk + 3].
__device__ __forceinline__ void buffer_quad(uint64_t seed, uint64_t blk, float z[4]) {
  const u32x4s r = philox4x32_10(u32x4s{(uint32_t)blk, 0u, 0u, kStreamBuffer}, (uint32_t)seed, (uint32_t)(seed >> 32));
  box_muller(r.x, r.y, &z[0], &z[1]);
  box_muller(r.z, r.w, &z[2], &z[3]);
}

__device__ __forceinline__ float buffer_value(uint64_t seed, uint64_t i) {
  float z[4];
  buffer_quad(seed, i >> 2, z);
  const uint32_t lane = (uint32_t)(i & 3);
  return lane == 0 ? z[0] : lane == 1 ? z[1] : lane == 2 ? z[2] : z[3];
}

// Jitter of the head-slab estimator: four Gaussians for draw g, token row r, columns 4 q .. 4 q + 3 (q < 64) of the
// jittered 256-column slab: philox(ctr = (64 r + q, g, 0, kStreamHead), key = seed), Box-Muller as above.
// Replaces the estimator's torch.randn draws (train/val/dust.py:192-193, 281).
__device__ __forceinline__ void head_noise_quad(uint64_t seed, uint32_t draw, uint32_t row, uint32_t q, float z[4]) {
  const u32x4s r = philox4x32_10(u32x4s{row * 64u + q, draw, 0u, kStreamHead}, (uint32_t)seed, (uint32_t)(seed >> 32));
  box_muller(r.x, r.y, &z[0], &z[1]);
  box_muller(r.z, r.w, &z[2], &z[3]);
}

// Jitter of the direct draws: four Gaussians for draw g at site s (0 token embedding, 1 attention output, 2 attention
// projection, 3 MLP hidden, 4 MLP projection), token row r (batch row * T + position), channels 4 q .. 4 q + 3 of a
// site `quads` * 4 channels wide: philox(ctr = (r * quads + q, g, s, kStreamDust), key = seed), Box-Muller as above.
// Replaces the direct draws' torch.randn (train/val/dust.py:192-193, 244).
__device__ __forceinline__ void dust_noise_quad(uint64_t seed, uint32_t draw, uint32_t site, uint32_t row,
                                                uint32_t quads, uint32_t q, float z[4]) {
  const u32x4s r =
      philox4x32_10(u32x4s{row * quads + q, draw, site, kStreamDust}, (uint32_t)seed, (uint32_t)(seed >> 32));
  box_muller(r.x, r.y, &z[0], &z[1]);
  box_muller(r.z, r.w, &z[2], &z[3]);
}

__device__ __forceinline__ int64_t offset_value(uint64_t seed, uint64_t step, uint32_t param, uint32_t direction,
                                                uint32_t range) {
  const uint64_t s = 1000003ull * seed + step;
  const u32x4s r = philox4x32_10(u32x4s{direction, param, 0u, kStreamOffset}, (uint32_t)s, (uint32_t)(s >> 32));
  return (int64_t)(((uint64_t)r.x * range) >> 32);
}

}  // namespace noise
