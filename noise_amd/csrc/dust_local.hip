// Dust's attention-internal estimates (train/val/dust.py:305-384): the decayed credit of later tokens' scores and the
// local draws' jitter.
//
// Decayed credit (dust.py:342-345, 378-381): out[r, t] = sum_{s = t}^{min(t + W, T - 1)} gamma^(s - t) score[r, s]
// for each row r = (o, i) of a [outer, T, inner] array (the reference's scores are [n, b, T, heads]: inner = heads),
// the reference's einsum of the scores with credit[t, s] = [0 <= s - t <= W] gamma^(s - t), in O(T) per row instead
// of a dense T x T matrix: with the untruncated suffix filter E[t] = score[t] + gamma E[t + 1] (E = 0 past the row),
// out[t] = E[t] - gamma^(W + 1) E[t + W + 1]. One workgroup of 256 threads per row: each thread runs the recurrence
// over its chunk of T / 256 consecutive positions, the chunks' carries go through a decayed suffix scan (lane shifts
// within a wave, then across the 4 waves), and the windowed difference reads E from LDS. A workgroup has read all of
// its row before it writes any of it, so out may be score itself.
#include <math.h>

#include "common.h"
#include "rng.h"

namespace noise {

constexpr int kDcMaxT = 8192;  // positions per row held in LDS

// score and out carry no __restrict__: out may be score itself (dust.decayed_credit calls it in place).
__global__ __launch_bounds__(256) void decayed_credit_kernel(const float* score, int T, int inner, int W, float gamma,
                                                             float* out) {
  __shared__ float e_s[kDcMaxT];
  __shared__ float suffix[256];
  __shared__ float wave_total[4];
  const int64_t r = blockIdx.x;
  const int64_t base = (r / inner) * T * inner + r % inner;  // element t of the row at base + t inner
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int C = T / 256;  // positions per thread (T % 256 == 0): chunk i = positions i C .. i C + C - 1
  const float* sr = score + base;
  const int t0 = tid * C;
  // the chunk's own suffix filter, back to front; a = its value at the chunk's first position
  float a = 0.f;
  for (int j = C - 1; j >= 0; --j) {
    a = fmaf(gamma, a, sr[(int64_t)(t0 + j) * inner]);
    e_s[t0 + j] = a;
  }
  // S_i = sum_{k >= i} g^(k - i) a_k with g = gamma^C: within a wave by doubling steps over the higher lanes ...
  const float g = powf(gamma, (float)C);
  float v = a, gp = g;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float up = __shfl_down(v, m, 64);
    if (lane + m < 64) v = fmaf(gp, up, v);
    gp *= gp;
  }
  if (lane == 0) wave_total[wave] = v;
  __syncthreads();
  // ... then the later waves, decayed to this wave's end: F = total of wave + 1 + g^64 (total of wave + 2 + ...)
  const float g64 = powf(gamma, (float)(64 * C));
  float later = 0.f;
  for (int w2 = 3; w2 > wave; --w2) later = fmaf(later, g64, wave_total[w2]);
  suffix[tid] = fmaf(later, powf(g, (float)(64 - lane)), v);
  __syncthreads();
  // E at the chunk's positions: own part + gamma^(C - j) E[t0 + C], E[t0 + C] = S of the next chunk
  const float after = tid < 255 ? suffix[tid + 1] : 0.f;
  for (int j = 0; j < C; ++j) e_s[t0 + j] = fmaf(powf(gamma, (float)(C - j)), after, e_s[t0 + j]);
  __syncthreads();
  const float gw = powf(gamma, (float)W + 1.f);
  for (int t = tid; t < T; t += 256) {
    const int64_t s = (int64_t)t + W + 1;
    out[base + (int64_t)t * inner] = s < T ? fmaf(-gw, e_s[s], e_s[t]) : e_s[t];
  }
}

// out[d, row, c] = the local draws' jitter of draw draw0 + d at `site`: rows x width values per draw (width % 4 == 0),
// the counter stream of the direct draws (rng.h dust_noise_quad).
__global__ __launch_bounds__(256) void dust_noise_kernel(uint64_t seed, uint32_t draw0, uint32_t site, int64_t rows,
                                                         int width, float* __restrict__ out) {
  const int quads = width / 4;
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;  // quad index within the draw
  if (i >= rows * quads) return;
  const uint32_t draw = draw0 + blockIdx.y;
  const int64_t row = i / quads;
  const int q = (int)(i % quads);
  float z[4];
  dust_noise_quad(seed, draw, site, (uint32_t)row, (uint32_t)quads, (uint32_t)q, z);
  *(f32x4*)(out + ((int64_t)blockIdx.y * rows + row) * width + 4 * q) = f32x4{z[0], z[1], z[2], z[3]};
}

// ---- the local draws (dust.py:339-382): the jittered operand, the per-head scores, the jitter-weighted estimate ----
// Rows are (draw j, batch row bi, token tt) in draw-major order, row index (j b + bi) t + tt; heads are 8 of 64
// channels. The jitter of draw j at `site` is the counter stream's (rng.h dust_noise_quad) over the token row bi t + tt,
// 512 channels wide (128 quads) for q, k, v, ve and 8 wide (2 quads) for the gate; nothing of it is stored.
enum LocalKind { kLocalRotary = 0, kLocalValue = 1, kLocalValueEmbed = 2, kLocalGate = 3 };

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + __expf(-x)); }

// One wave per row: lane l takes head l / 8 and its channels 4 (l % 8) .. + 3 and their rotary partners 32 higher.
//   kLocalRotary:     out = bf16(norm(rotary(raw + sigma a)))  (dust.py:324-325, 352-355; raw = the clean q or k)
//   kLocalValue:      out = bf16(sigma a)                       (dust.py:369)
//   kLocalValueEmbed: out = bf16(sigma a 2 sigmoid(z_h))        (dust.py:370-371)
//   kLocalGate:       out = bf16((2 sigmoid(z_h + sigma a_h) - 2 sigmoid(z_h - sigma a_h)) ve)  (dust.py:364-367)
__global__ __launch_bounds__(256) void local_operand_kernel(int kind, uint64_t seed, uint32_t draw0, uint32_t site,
                                                            int b, int t, const bf16_t* __restrict__ raw,
                                                            const bf16_t* __restrict__ z, const float* __restrict__ ve,
                                                            const float* __restrict__ cosv, const float* __restrict__ sinv,
                                                            float sigma, int64_t rows, bf16_t* __restrict__ out) {
#pragma clang fp contract(off)
  const int64_t row = blockIdx.x * 4ll + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63, h = lane >> 3, sub = lane & 7;
  const int64_t bt = (int64_t)b * t;
  const int j = (int)(row / bt);
  const int64_t tok = row % bt;  // bi t + tt
  const int tt = (int)(tok % t);
  const int c_lo = 64 * h + 4 * sub, c_hi = c_lo + 32;
  float lo[4], hi[4];
  const uint32_t draw = draw0 + (uint32_t)j;
  if (kind == kLocalGate) {
    float g[4];
    dust_noise_quad(seed, draw, site, (uint32_t)tok, 2u, (uint32_t)(h >> 2), g);
    const float ah = g[h & 3], zh = bf16_to_f32(z[tok * 8 + h]);
    const float dg = 2.0f * sigmoid_f(zh + sigma * ah) - 2.0f * sigmoid_f(zh - sigma * ah);
    const float* vr = ve + tok * 512;
#pragma unroll
    for (int e = 0; e < 4; ++e) { lo[e] = dg * vr[c_lo + e]; hi[e] = dg * vr[c_hi + e]; }
  } else {
    float alo[4], ahi[4];
    dust_noise_quad(seed, draw, site, (uint32_t)tok, 128u, (uint32_t)(c_lo >> 2), alo);
    dust_noise_quad(seed, draw, site, (uint32_t)tok, 128u, (uint32_t)(c_hi >> 2), ahi);
    if (kind == kLocalRotary) {
      const bf16_t* rr = raw + tok * 512;
      float x1[4], x2[4], ss = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x1[e] = bf16_to_f32(rr[c_lo + e]) + sigma * alo[e];
        x2[e] = bf16_to_f32(rr[c_hi + e]) + sigma * ahi[e];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float cs = cosv[tt * 32 + 4 * sub + e], sn = sinv[tt * 32 + 4 * sub + e];
        lo[e] = x1[e] * cs + x2[e] * sn;
        hi[e] = x1[e] * -sn + x2[e] * cs;
        ss += lo[e] * lo[e];
        ss += hi[e] * hi[e];
      }
      // the head's 64 channels sit in lanes 8 h .. 8 h + 7
      ss += __shfl_xor(ss, 1, 64);
      ss += __shfl_xor(ss, 2, 64);
      ss += __shfl_xor(ss, 4, 64);
      const float inv = 1.0f / __builtin_sqrtf(ss / 64.0f + 1.1920928955078125e-07f);
#pragma unroll
      for (int e = 0; e < 4; ++e) { lo[e] *= inv; hi[e] *= inv; }
    } else {  // (sigma a), times 2 sigmoid(z_h) for the value embedding
      const float g = kind == kLocalValueEmbed ? 2.0f * sigmoid_f(bf16_to_f32(z[tok * 8 + h])) : 1.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo[e] = (sigma * alo[e]) * g;
        hi[e] = (sigma * ahi[e]) * g;
      }
    }
  }
  bf16_t* o = out + row * 512;
  *(u32x2*)(o + c_lo) = u32x2{pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3])};
  *(u32x2*)(o + c_hi) = u32x2{pack_bf16x2(hi[0], hi[1]), pack_bf16x2(hi[2], hi[3])};
}

// score[row, h] = sum over head h's 64 channels of target[bi, tt] . (att[row] - baseline[bi, tt]) (baseline NULL: att
// itself); att and baseline bf16, target and the products fp32 (dust.py:375-377). One wave per row, 8 lanes per head.
__global__ __launch_bounds__(256) void local_score_kernel(const bf16_t* __restrict__ att,
                                                          const bf16_t* __restrict__ baseline,
                                                          const float* __restrict__ target, int64_t bt, int64_t rows,
                                                          float* __restrict__ score) {
  const int64_t row = blockIdx.x * 4ll + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t tok = row % bt;
  const int c0 = 8 * lane;  // 8 channels of head lane / 8
  const u32x4 av = *(const u32x4*)(att + row * 512 + c0);
  u32x4 bv = u32x4{0u, 0u, 0u, 0u};
  if (baseline) bv = *(const u32x4*)(baseline + tok * 512 + c0);
  const f32x4 t0 = *(const f32x4*)(target + tok * 512 + c0), t1 = *(const f32x4*)(target + tok * 512 + c0 + 4);
  float acc = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float d_lo = __uint_as_float(av[w] << 16) - __uint_as_float(bv[w] << 16);
    const float d_hi = __uint_as_float(av[w] & 0xFFFF0000u) - __uint_as_float(bv[w] & 0xFFFF0000u);
    const float ta = w < 2 ? t0[2 * w] : t1[2 * w - 4], tb = w < 2 ? t0[2 * w + 1] : t1[2 * w - 3];
    acc = fmaf(ta, d_lo, acc);
    acc = fmaf(tb, d_hi, acc);
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 4, 64);
  if ((lane & 7) == 0) score[row * 8 + (lane >> 3)] = acc;
}

// err[bi, tt, c] += sum_j score[(j b + bi) t + tt, head of c] a_j[bi, tt, c] * inv_divisor over the chunk's n draws,
// the jitter regenerated (dust.py:378-382). One thread per (token row, quad of channels); width 512 or 8 (the gate).
__global__ __launch_bounds__(256) void local_estimate_kernel(const float* __restrict__ score, uint64_t seed,
                                                             uint32_t draw0, uint32_t site, int n, int64_t bt,
                                                             int width, float inv_divisor, float* __restrict__ err) {
  const int quads = width / 4;
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= bt * quads) return;
  const int64_t tok = i / quads;
  const int q = (int)(i % quads);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < n; ++j) {
    float a[4];
    dust_noise_quad(seed, draw0 + (uint32_t)j, site, (uint32_t)tok, (uint32_t)quads, (uint32_t)q, a);
    const float* sr = score + ((int64_t)j * bt + tok) * 8;
    if (width == 8) {  // the gate: channel = head
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(sr[4 * q + e], a[e], acc[e]);
    } else {
      const float s = sr[q >> 4];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(s, a[e], acc[e]);
    }
  }
  f32x4* o = (f32x4*)(err + tok * width + 4 * q);
  f32x4 v = *o;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] += acc[e] * inv_divisor;
  *o = v;
}

}  // namespace noise

using namespace noise;

extern "C" int noise_decayed_credit(const float* score, int64_t outer, int64_t T, int32_t inner, int32_t window,
                                    float gamma, float* out, void* stream) {
  NOISE_REQUIRE(score && out, "NULL pointer argument");
  NOISE_REQUIRE(inner > 0 && outer > 0 && outer * inner <= INT32_MAX, "outer, inner positive, outer * inner < 2^31");
  NOISE_REQUIRE(T > 0 && T % 256 == 0 && T <= kDcMaxT, "T = %lld must be a multiple of 256 and at most %d",
                (long long)T, kDcMaxT);
  NOISE_REQUIRE(window >= 0, "negative window");
  NOISE_REQUIRE(gamma > 0.f && gamma < 1.f, "gamma must lie in (0, 1)");
  hipLaunchKernelGGL(decayed_credit_kernel, dim3((unsigned)(outer * inner)), dim3(256), 0, (hipStream_t)stream, score,
                     (int)T, (int)inner, window, gamma, out);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" int noise_dust_noise(uint64_t seed, uint32_t draw0, uint32_t site, int32_t n_draws, int64_t rows,
                                int32_t width, float* out, void* stream) {
  NOISE_REQUIRE(out, "NULL pointer argument");
  NOISE_REQUIRE(n_draws > 0 && n_draws <= 65535, "n_draws outside [1, 65535]");
  NOISE_REQUIRE(rows > 0 && width > 0 && width % 4 == 0 && rows * (width / 4) <= (int64_t)INT32_MAX,
                "rows > 0 and width a positive multiple of 4 required");
  const int64_t quads = rows * (width / 4);
  hipLaunchKernelGGL(dust_noise_kernel, dim3((unsigned)((quads + 255) / 256), (unsigned)n_draws), dim3(256), 0,
                     (hipStream_t)stream, seed, draw0, site, rows, (int)width, out);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" int noise_local_operand(int32_t kind, uint64_t seed, uint32_t draw0, uint32_t site, int32_t n_draws,
                                   int32_t b, int32_t t, const uint16_t* raw, const uint16_t* z, const float* ve,
                                   const float* cos_table, const float* sin_table, float sigma, uint16_t* out,
                                   void* stream) {
  NOISE_REQUIRE(out, "NULL output");
  NOISE_REQUIRE(kind >= 0 && kind <= 3, "kind %d outside 0..3", kind);
  NOISE_REQUIRE(n_draws > 0 && b > 0 && t > 0, "n_draws, b and t must be positive");
  NOISE_REQUIRE(kind != kLocalRotary || (raw && cos_table && sin_table), "the rotary kind needs raw, cos and sin");
  NOISE_REQUIRE(kind < kLocalValueEmbed || z, "ve and gate need z");
  NOISE_REQUIRE(kind != kLocalGate || ve, "the gate needs ve");
  NOISE_REQUIRE((int64_t)b * t <= (int64_t)UINT32_MAX, "b * t token rows exceed the counter stream's row field");
  const int64_t rows = (int64_t)n_draws * b * t;
  NOISE_REQUIRE((rows + 3) / 4 <= (int64_t)UINT32_MAX, "too many rows");
  hipLaunchKernelGGL(local_operand_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, kind,
                     seed, draw0, site, b, t, (const bf16_t*)raw, (const bf16_t*)z, ve, cos_table, sin_table, sigma,
                     rows, (bf16_t*)out);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" int noise_local_score(const uint16_t* att, const uint16_t* baseline, const float* target, int32_t n_draws,
                                 int32_t b, int32_t t, float* score, void* stream) {
  NOISE_REQUIRE(att && target && score, "NULL pointer argument");
  NOISE_REQUIRE(n_draws > 0 && b > 0 && t > 0, "n_draws, b and t must be positive");
  const int64_t bt = (int64_t)b * t, rows = bt * n_draws;
  NOISE_REQUIRE((rows + 3) / 4 <= (int64_t)UINT32_MAX, "too many rows");
  hipLaunchKernelGGL(local_score_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)att, (const bf16_t*)baseline, target, bt, rows, score);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" int noise_local_estimate(const float* score, uint64_t seed, uint32_t draw0, uint32_t site, int32_t n_draws,
                                    int32_t b, int32_t t, int32_t width, float inv_divisor, float* err, void* stream) {
  NOISE_REQUIRE(score && err, "NULL pointer argument");
  NOISE_REQUIRE(n_draws > 0 && b > 0 && t > 0, "n_draws, b and t must be positive");
  NOISE_REQUIRE(width == 512 || width == 8, "width must be 512 (q, k, v, ve) or 8 (the gate)");
  const int64_t bt = (int64_t)b * t, threads = bt * (width / 4);
  NOISE_REQUIRE(bt <= (int64_t)UINT32_MAX && (threads + 255) / 256 <= (int64_t)UINT32_MAX, "too many token rows");
  hipLaunchKernelGGL(local_estimate_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     score, seed, draw0, site, (int)n_draws, bt, (int)width, inv_divisor, err);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}
