// Dust's estimators that need no forward pass of their own: the head-slab CE estimator (train/val/dust.py:261-303,
// DUST.head_error), and the reward and error sums of the direct draws (dust.py:235-259, DUST.direct_errors; their
// reruns are the population forward's kernels, forward.hip noise_dust_rerun).
//
// Head-slab estimator: per-token error estimates of the lm_head outputs from draws that jitter one 256-column
// vocabulary slab at a time.
//
// For chunk c of n draws (n = the largest count <= nrep dividing draws) the jittered slab is c % slabs. Draw g of the
// chunk changes the slab's capped logits to 15 tanh((raw + sigma a_g) / 15) and recomputes the token's CE from the
// cached exponential sums of the other slabs. The reward is the clean loss minus that CE (0 at ignored targets),
// centered over the batch when b > 1. The error of the slab's columns is -(sum over its draws of reward / sigma * a)
// / (draws per slab); columns past the vocabulary are 0.
//
// Four launches, all of them element-parallel:
//   head_prep_kernel    one wave per token row: capped logits, the 16 slab sums of exp, their total, the target logit
//   head_loss_kernel    one wave per (draw, row): the 256 jittered columns (4 per lane, one Philox call), the CE
//   head_center_kernel  one thread per (draw, position): rewards, centered over the batch
//   head_accum_kernel   one wave per (row, slab): the draws of that slab regenerate their jitter, the error sum
// The jitter is this library's counter stream (rng.h head_noise_quad), never stored.
//
// Direct draws, per chunk of n draws: dust_reward_kernel (clean minus perturbed per-token loss, centered over the
// draws), dust_rtg_kernel (gamma > 0: the decayed reward-to-go along the sequence), dust_accum_kernel (one thread per
// token row and 4 channels of the site: the n draws' jitter regenerated (rng.h dust_noise_quad), error -= sum of
// reward / sigma * a).
#include <math.h>

#include "common.h"
#include "rng.h"

namespace noise {

constexpr int kSlab = 256;

__device__ __forceinline__ float soft_cap(float x) { return 15.0f * tanhf(x / 15.0f); }

// 4 bf16 (8 bytes) as floats
__device__ __forceinline__ f32x4 ld_bf16x4(const bf16_t* p) {
  const u32x2 q = *(const u32x2*)p;
  return f32x4{bf16_lo(q[0]), bf16_hi(q[0]), bf16_lo(q[1]), bf16_hi(q[1])};
}

__global__ __launch_bounds__(256) void head_prep_kernel(const bf16_t* __restrict__ raw, int64_t ld,
                                                        const int64_t* __restrict__ targets, int64_t rows, int slabs,
                                                        float* __restrict__ slab_sums, float* __restrict__ total,
                                                        float* __restrict__ clean_t) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bf16_t* r = raw + row * ld;
  const int64_t tg0 = targets[row];
  const int tg = tg0 < 0 ? 0 : (int)tg0;  // the reference clamps ignored targets to 0 (dust.py:275)
  float tot = 0.f, tz = 0.f;
  for (int s = 0; s < slabs; ++s) {
    const int c0 = s * kSlab + 4 * lane;
    const f32x4 x = ld_bf16x4(r + c0);
    float e = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float z = soft_cap(x[k]);
      e += expf(z);
      if (c0 + k == tg) tz = z;
    }
    const float se = warp_sum(e);
    if (lane == 0) slab_sums[row * slabs + s] = se;
    tot += se;
  }
  tz = warp_sum(tz);  // one lane holds the target logit, the others 0
  if (lane == 0) {
    total[row] = tot;
    clean_t[row] = tz;
  }
}

__global__ __launch_bounds__(256) void head_loss_kernel(const bf16_t* __restrict__ raw, int64_t ld,
                                                        const int64_t* __restrict__ targets, int64_t rows, int slabs,
                                                        int n, float sigma, uint64_t seed,
                                                        const float* __restrict__ slab_sums,
                                                        const float* __restrict__ total,
                                                        const float* __restrict__ clean_t, float* __restrict__ loss) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const uint32_t g = blockIdx.y;  // draw
  if (row >= rows) return;
  const int block = (int)(g / (uint32_t)n) % slabs, lo = block * kSlab;
  float a[4];
  head_noise_quad(seed, g, (uint32_t)row, (uint32_t)lane, a);
  const f32x4 x = ld_bf16x4(raw + row * ld + lo + 4 * lane);
  const int64_t tg0 = targets[row];
  const int tg = tg0 < 0 ? 0 : (int)tg0;
  float e = 0.f, tz = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float z = soft_cap(x[k] + sigma * a[k]);
    e += expf(z);
    if (lo + 4 * lane + k == tg) tz = z;
  }
  e = warp_sum(e);
  tz = warp_sum(tz);
  if (lane == 0) {
    const float part = (total[row] - slab_sums[row * slabs + block]) + e;
    const bool in_slab = tg >= lo && tg < lo + kSlab;
    loss[(int64_t)g * rows + row] = logf(part) - (in_slab ? tz : clean_t[row]);
  }
}

// reward[g, r] = (target[r] != -1) ? clean[r] - loss[g, r] : 0, minus its mean over the batch (rows bi * t + ti)
__global__ __launch_bounds__(256) void head_center_kernel(const int64_t* __restrict__ targets,
                                                          const float* __restrict__ clean, int b, int t, int draws,
                                                          float* __restrict__ loss) {
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= (int64_t)draws * t) return;
  const int64_t g = id / t, ti = id % t, rows = (int64_t)b * t;
  float* lg = loss + g * rows;
  float mean = 0.f;
  for (int bi = 0; bi < b; ++bi) {
    const int64_t r = (int64_t)bi * t + ti;
    const float rw = targets[r] != -1 ? clean[r] - lg[r] : 0.f;
    lg[r] = rw;
    mean += rw;
  }
  if (b > 1) {
    mean /= (float)b;
    for (int bi = 0; bi < b; ++bi) lg[(int64_t)bi * t + ti] -= mean;
  }
}

__global__ __launch_bounds__(256) void head_accum_kernel(const float* __restrict__ reward, int64_t rows, int64_t ld,
                                                         int slabs, int n_slab_ld, int n, int chunks, float sigma,
                                                         float inv_per_slab, uint64_t seed,
                                                         float* __restrict__ error) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= rows * n_slab_ld) return;
  const int64_t row = w / n_slab_ld;
  const int slab = (int)(w % n_slab_ld), c0 = slab * kSlab + 4 * lane;
  float* out = error + row * ld;
  if (slab >= slabs) {  // past the vocabulary
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (c0 + k < ld) out[c0 + k] = 0.f;
    return;
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c = slab; c < chunks; c += slabs)
    for (int j = 0; j < n; ++j) {
      const uint32_t g = (uint32_t)(c * n + j);
      const float wgt = reward[(int64_t)g * rows + row] / sigma;
      float a[4];
      head_noise_quad(seed, g, (uint32_t)row, (uint32_t)lane, a);
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[k] += wgt * a[k];
    }
  *(f32x4*)(out + c0) = f32x4{-acc[0] * inv_per_slab, -acc[1] * inv_per_slab, -acc[2] * inv_per_slab,
                              -acc[3] * inv_per_slab};
}

// reward[j, r] = clean[r] - loss[j, r], minus its mean over the chunk's n draws (n > 1) (dust.py:246-249)
__global__ __launch_bounds__(256) void dust_reward_kernel(const float* __restrict__ loss, const float* __restrict__ clean,
                                                          int n, int64_t rows, float* __restrict__ reward) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const float c = clean[r];
  float mean = 0.f;
  for (int j = 0; j < n; ++j) {
    const float rw = c - loss[(int64_t)j * rows + r];
    reward[(int64_t)j * rows + r] = rw;
    mean += rw;
  }
  if (n > 1) {
    mean /= (float)n;
    for (int j = 0; j < n; ++j) reward[(int64_t)j * rows + r] -= mean;
  }
}

// out[s, t] = sum_{k < lags, t + k < T} gamma^k reward[s, t + k] for each of the n_seqs sequences (dust.py:86-91)
__global__ __launch_bounds__(256) void dust_rtg_kernel(const float* __restrict__ reward, int64_t n_seqs, int T,
                                                       float gamma, int lags, float* __restrict__ out) {
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= n_seqs * T) return;
  const int64_t s = id / T;
  const int t = (int)(id % T);
  const float* r = reward + s * T;
  float acc = 0.f, g = 1.f;
  for (int k = 0; k < lags && t + k < T; ++k) {
    acc += g * r[t + k];
    g *= gamma;
  }
  out[id] = acc;
}

// error[r, 4 q ..] -= sum_j reward[j, r] / sigma * a_j[r, 4 q ..]: one thread per token row r and 4 channels q
__global__ __launch_bounds__(256) void dust_accum_kernel(const float* __restrict__ reward, int n, int64_t rows,
                                                         int quads, float sigma, uint64_t seed, int draw0,
                                                         uint32_t site, float* __restrict__ error) {
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= rows * quads) return;
  const int64_t r = id / quads;
  const int q = (int)(id % quads);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < n; ++j) {
    const float w = reward[(int64_t)j * rows + r] / sigma;
    float a[4];
    dust_noise_quad(seed, (uint32_t)(draw0 + j), site, (uint32_t)r, (uint32_t)quads, (uint32_t)q, a);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] += w * a[k];
  }
  f32x4* e = (f32x4*)(error + r * (int64_t)quads * 4 + 4 * q);
  const f32x4 old = *e;
  *e = f32x4{old[0] - acc[0], old[1] - acc[1], old[2] - acc[2], old[3] - acc[3]};
}

static inline size_t al256h(size_t n) { return (n + 255) & ~(size_t)255; }

static int chunk_of(int draws, int cap) {
  for (int n = cap < draws ? cap : draws; n > 0; --n)
    if (draws % n == 0) return n;
  return 1;
}

}  // namespace noise

using namespace noise;

extern "C" size_t noise_head_error_workspace(int64_t rows, int32_t vocab, int32_t draws) {
  const int slabs = vocab / kSlab;
  return al256h((size_t)rows * slabs * 4) + 2 * al256h((size_t)rows * 4) + al256h((size_t)draws * rows * 4);
}

extern "C" int noise_head_error(const uint16_t* raw, int64_t ld, const int64_t* targets, const float* clean_loss,
                                int32_t b, int32_t t, int32_t vocab, int32_t draws, int32_t nrep, float sigma,
                                uint64_t seed, float* error, void* workspace, size_t workspace_bytes, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  NOISE_REQUIRE(raw && targets && clean_loss && error, "NULL pointer argument");
  NOISE_REQUIRE(b > 0 && t > 0, "b and t must be positive");
  NOISE_REQUIRE(vocab > 0 && vocab % kSlab == 0 && vocab <= ld && ld % 4 == 0,
                "vocab = %d must be a positive multiple of 256, at most ld = %lld (a multiple of 4)", vocab,
                (long long)ld);
  NOISE_REQUIRE(draws > 0 && nrep > 0 && sigma > 0.f, "draws, nrep and sigma must be positive");
  const int64_t rows = (int64_t)b * t;
  NOISE_REQUIRE(rows <= (1ll << 26), "b * t = %lld exceeds 2^26 token rows", (long long)rows);
  NOISE_REQUIRE((int64_t)draws * rows <= (1ll << 40), "draws * rows too large");
  const int slabs = vocab / kSlab, n = chunk_of(draws, nrep), chunks = draws / n;
  NOISE_REQUIRE(chunks % slabs == 0, "the %d chunks of %d draws must cover the %d slabs evenly", chunks, n, slabs);
  NOISE_REQUIRE(draws <= 65535, "draws = %d exceeds one launch's grid (65,535)", draws);
  NOISE_REQUIRE(workspace && workspace_bytes >= noise_head_error_workspace(rows, vocab, draws), "workspace too small");
  char* p = (char*)workspace;
  float* slab_sums = (float*)p;
  p += al256h((size_t)rows * slabs * 4);
  float* total = (float*)p;
  p += al256h((size_t)rows * 4);
  float* clean_t = (float*)p;
  p += al256h((size_t)rows * 4);
  float* loss = (float*)p;
  const unsigned row_blocks = (unsigned)((rows + 3) / 4);
  const bf16_t* r = (const bf16_t*)raw;
  NoiseTimer tm(kTimeHeadError, stream);
  hipLaunchKernelGGL(head_prep_kernel, dim3(row_blocks), dim3(256), 0, stream, r, ld, targets, rows, slabs, slab_sums,
                     total, clean_t);
  NOISE_LAUNCH_CHECK();
  hipLaunchKernelGGL(head_loss_kernel, dim3(row_blocks, (unsigned)draws), dim3(256), 0, stream, r, ld, targets, rows,
                     slabs, n, sigma, seed, slab_sums, total, clean_t, loss);
  NOISE_LAUNCH_CHECK();
  const int64_t nct = (int64_t)draws * t;
  hipLaunchKernelGGL(head_center_kernel, dim3((unsigned)((nct + 255) / 256)), dim3(256), 0, stream, targets,
                     clean_loss, b, t, draws, loss);
  NOISE_LAUNCH_CHECK();
  const int n_slab_ld = (int)((ld + kSlab - 1) / kSlab);
  const int64_t waves = rows * n_slab_ld;
  hipLaunchKernelGGL(head_accum_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, loss, rows, ld, slabs,
                     n_slab_ld, n, chunks, sigma, 1.0f / (float)(draws / slabs), seed, error);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" size_t noise_dust_errors_workspace(int32_t n_draws, int64_t n_seq, int64_t T) {
  if (n_draws <= 0 || n_seq <= 0 || T <= 0) return 0;
  return 2 * al256h((size_t)n_draws * n_seq * T * 4);
}

extern "C" int noise_dust_errors(const float* token_loss, const float* clean_loss, int32_t n_draws, int64_t n_seq,
                                 int64_t T, float gamma, float sigma, uint64_t seed, int32_t draw0, int32_t site,
                                 int32_t width, float* error, void* workspace, size_t workspace_bytes,
                                 void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  NOISE_REQUIRE(token_loss && clean_loss && error, "NULL pointer argument");
  NOISE_REQUIRE(n_draws > 0 && n_seq > 0 && T > 0 && draw0 >= 0, "n_draws, n_seq, T positive and draw0 >= 0 needed");
  NOISE_REQUIRE(sigma > 0.f && gamma >= 0.f && gamma < 1.f, "sigma > 0 and 0 <= gamma < 1 needed");
  NOISE_REQUIRE(site >= 0 && site <= 4 && width > 0 && width % 4 == 0, "site %d outside [0, 4] or width %d not a "
                "positive multiple of 4", site, width);
  const int64_t rows = n_seq * T;
  NOISE_REQUIRE(rows * (width / 4) <= ((int64_t)1 << 32) - 1, "rows * width / 4 exceeds the jitter counter");
  NOISE_REQUIRE(workspace && workspace_bytes >= noise_dust_errors_workspace(n_draws, n_seq, T), "workspace too small");
  float* reward = (float*)workspace;
  float* rtg = (float*)((char*)workspace + al256h((size_t)n_draws * rows * 4));
  NoiseTimer tm(kTimeDustErrors, stream);
  hipLaunchKernelGGL(dust_reward_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, token_loss,
                     clean_loss, n_draws, rows, reward);
  NOISE_LAUNCH_CHECK();
  const float* w = reward;
  if (gamma > 0.f) {
    const int lags = (int)ceil(log(1e-6) / log((double)gamma));
    const int64_t n_el = (int64_t)n_draws * rows;
    hipLaunchKernelGGL(dust_rtg_kernel, dim3((unsigned)((n_el + 255) / 256)), dim3(256), 0, stream, reward,
                       (int64_t)n_draws * n_seq, (int)T, gamma, lags, rtg);
    NOISE_LAUNCH_CHECK();
    w = rtg;
  }
  const int quads = width / 4;
  const int64_t threads = rows * quads;
  hipLaunchKernelGGL(dust_accum_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, w, n_draws,
                     rows, quads, sigma, seed, draw0, (uint32_t)site, error);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}
