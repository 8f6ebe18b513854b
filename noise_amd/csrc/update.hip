// Fitness, gradient assembly and the AdamW step of the EGGROLL update
// (archive/10M/train/val/eggroll.py:151-167; optimizer semantics of torch.optim.AdamW as built at :205).
#include <math.h>
#include <string.h>

#include "common.h"

namespace noise {

// One workgroup: f_j = L[2j+1] - L[2j]; f /= (unbiased std + 1e-8); weight[d] = sum_{j % pairs == d} f_j in j order.
__global__ __launch_bounds__(1024) void fitness_kernel(const float* __restrict__ losses, int64_t n, int64_t pairs,
                                                       float* __restrict__ fitness, float* __restrict__ weight) {
  __shared__ float red[16];
  __shared__ float stat[2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float s = 0.f;
  for (int64_t j = tid; j < n; j += 1024) s += losses[2 * j + 1] - losses[2 * j];
  s = warp_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int w = 0; w < 16; ++w) t += red[w];
    stat[0] = t / (float)n;
  }
  __syncthreads();
  const float mean = stat[0];
  float q = 0.f;
  for (int64_t j = tid; j < n; j += 1024) {
    const float d = (losses[2 * j + 1] - losses[2 * j]) - mean;
    q += d * d;
  }
  q = warp_sum(q);
  __syncthreads();
  if (lane == 0) red[wave] = q;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int w = 0; w < 16; ++w) t += red[w];
    const float sd = n > 1 ? sqrtf(t / (float)(n - 1)) : __builtin_nanf("");
    stat[1] = 1.0f / (sd + 1e-8f);
  }
  __syncthreads();
  const float inv = stat[1];
  for (int64_t j = tid; j < n; j += 1024) fitness[j] = (losses[2 * j + 1] - losses[2 * j]) * inv;
  for (int64_t d = tid; d < pairs; d += 1024) {
    float w = 0.f;
    for (int64_t j = d; j < n; j += pairs) w += (losses[2 * j + 1] - losses[2 * j]) * inv;
    weight[d] = w;
  }
}

// grad[o, i] = scale sum_j w_j a_j[o] b_j[i] (eggroll.py:159-161: (w a)^T b over the pairs), on fp32 MFMA
// (v_mfma_f32_32x32x2_f32, full fp32 products and sums). A workgroup owns a 128 x 128 output tile, each of its 4 waves
// 64 x 64 (2 x 2 MFMA tiles); the pairs stream through two LDS stages of 16: a_j[o0 .. o0+127] and w_j b_j[i0 ..]
// as rows [pair][128] padded to 160 floats, so the two pair rows of one operand read (lanes 0..31 and 32..63) fall
// in opposite halves of the 64 banks. Every load is a 256-byte row segment (thread: one column, 8 of the 16 rows);
// columns past out / in and pairs past the last read as zeros, so offsets and sizes need no alignment.
// One launch covers a list of matrices (jobs, by value in the kernel arguments): the launch's tiles are numbered job by
// job, each job's in row-major order over ceil(out / 128) x ceil(in / 128); tile t belongs to the job whose range
// [tile0, next tile0) holds it, and each XCD takes a contiguous run of tile numbers.
constexpr int kOgTile = 128, kOgK = 16, kOgPitch = 160, kOgMaxJobs = 64;

struct OgJob {
  int64_t a_off, b_off;  // column offsets of a (out values) and b (in values) in their rows
  int32_t out, in;
  int32_t tile0, n_in_tiles;
  float* grad;           // [out, in]
};
struct OgJobs {
  int32_t n;
  int32_t accumulate;  // add to the gradients instead of overwriting them
  int32_t total;       // tiles of the launch (the grid is that rounded up to a multiple of 8)
  OgJob job[kOgMaxJobs];
};

// Sum over k < n_k of a_k b_k^T with row k of A at a_rows + k a_stride (fp32) and of B at b_rows + k b_stride (fp32,
// or bf16 with b_bf16), b_k scaled by weight[k] when a weight is given.
__global__ __launch_bounds__(256) void outer_grad_kernel(const float* __restrict__ a_rows, int64_t a_stride,
                                                         const void* __restrict__ b_rows, int64_t b_stride, int b_bf16,
                                                         const float* __restrict__ weight, int64_t pairs, float scale,
                                                         OgJobs jobs) {
  __shared__ float as[2][kOgK][kOgPitch];
  __shared__ float bs[2][kOgK][kOgPitch];
  // Workgroups are dispatched round-robin over the 8 XCDs; XCD x takes the contiguous tile range
  // [x per, (x + 1) per), so the tiles of one matrix, which read the same a and b slices, share one L2.
  const int per = (int)(gridDim.x / 8);
  const int tid_ = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (tid_ >= jobs.total) return;  // the grid's round-up
  int jb = 0;
  while (jb + 1 < jobs.n && tid_ >= jobs.job[jb + 1].tile0) ++jb;
  const OgJob& job = jobs.job[jb];
  const int64_t a_off = job.a_off, b_off = job.b_off, out = job.out, in = job.in;
  float* __restrict__ grad = job.grad;
  const int tile = tid_ - job.tile0;
  const int64_t o0 = (int64_t)(tile / job.n_in_tiles) * kOgTile, i0 = (int64_t)(tile % job.n_in_tiles) * kOgTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wo = (wave >> 1) * 64, wi = (wave & 1) * 64;
  const int col = tid & 127, row0 = tid >> 7;  // loader: column col of rows row0, row0 + 2, ..., row0 + 14
  const bool a_in = o0 + col < out, b_in = i0 + col < in;

  float ra[8], rb[8];
  auto load = [&](int64_t j0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t j = j0 + row0 + 2 * q;
      const bool live = j < pairs;
      const int64_t jj = live ? j : 0;
      ra[q] = (live && a_in) ? a_rows[jj * a_stride + a_off + o0 + col] : 0.f;
      float bv = 0.f;
      if (live && b_in) {
        const int64_t at = jj * b_stride + b_off + i0 + col;
        bv = b_bf16 ? bf16_to_f32(((const bf16_t*)b_rows)[at]) : ((const float*)b_rows)[at];
        if (weight) bv = weight[j] * bv;
      }
      rb[q] = bv;
    }
  };
  auto store = [&](int st) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      as[st][row0 + 2 * q][col] = ra[q];
      bs[st][row0 + 2 * q][col] = rb[q];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int v = 0; v < 2; ++v)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[u][v][r] = 0.f;

  load(0);
  store(0);
  __syncthreads();
  const int64_t n_steps = (pairs + kOgK - 1) / kOgK;
  const int kr = lane >> 5, lc = lane & 31;  // operand lane: pair row kr of the k pair, column lc of the 32
  for (int64_t t = 0; t < n_steps; ++t) {
    const int st = (int)(t & 1);
    const bool more = t + 1 < n_steps;
    if (more) load((t + 1) * kOgK);
#pragma unroll
    for (int s = 0; s < kOgK / 2; ++s) {
      float fa[2], fb[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        fa[u] = as[st][2 * s + kr][wo + 32 * u + lc];
        fb[u] = bs[st][2 * s + kr][wi + 32 * u + lc];
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int v = 0; v < 2; ++v) acc[u][v] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[u], fb[v], acc[u][v], 0, 0, 0);
    }
    if (more) store(st ^ 1);
    __syncthreads();
  }

  // accumulator register r of tile (u, v): row 8 (r / 4) + 4 (lane / 32) + r % 4, column lane % 32
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int v = 0; v < 2; ++v)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t o = o0 + wo + 32 * u + 8 * (r >> 2) + 4 * kr + (r & 3), i = i0 + wi + 32 * v + lc;
        if (o < out && i < in) {
          float* gp = grad + o * in + i;
          *gp = jobs.accumulate ? fmaf(scale, acc[u][v][r], *gp) : scale * acc[u][v][r];
        }
      }
}

// grad[i] = scale sum_j w_j eps_j[i] (1-D parameters: eggroll.py:163). A block owns 8 consecutive elements; its 256
// threads take the pairs j = t, t + 256, ... and a fixed-order tree in LDS adds their partial sums (deterministic).
__global__ __launch_bounds__(256) void vector_grad_kernel(const float* __restrict__ rows, int64_t stride, int64_t a_off,
                                                          const float* __restrict__ weight, int64_t pairs, int64_t n,
                                                          float scale, int accumulate, float* __restrict__ grad) {
  __shared__ float red[256][9];
  const int tid = threadIdx.x;
  const int64_t i0 = (int64_t)blockIdx.x * 8;
  float acc[8] = {};
  for (int64_t j = tid; j < pairs; j += 256) {
    const float wj = weight[j];
    const float* row = rows + j * stride + a_off + i0;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (i0 + e < n) acc[e] += wj * row[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[tid][e] = acc[e];
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (tid < w)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[tid][e] += red[tid + w][e];
    __syncthreads();
  }
  if (tid < 8 && i0 + tid < n)
    grad[i0 + tid] = accumulate ? fmaf(scale, red[0][tid], grad[i0 + tid]) : scale * red[0][tid];
}

struct AdamScalars {
  float lr_wd;       // 1 - lr * weight_decay
  float one_m_b1;    // lerp weight
  float b2, one_m_b2;
  float neg_step_size;  // -lr / (1 - b1^step)
  float bc2_sqrt;       // sqrt(1 - b2^step)
  float eps;
};

// torch.optim.AdamW (foreach path) on one element: p *= 1 - lr wd; m = lerp(m, g, 1 - b1); v = v b2 + (1 - b2) g g;
// p += -step_size * m / (sqrt(v) / bc2_sqrt + eps).
__device__ __forceinline__ void adam_element(float& p, float g, float& m, float& v, const AdamScalars& s) {
  p = p * s.lr_wd;
  // torch's lerp: weight < 0.5 ? start + w (end - start) : end - (end - start) (1 - w)
  m = (s.one_m_b1 < 0.5f) ? m + s.one_m_b1 * (g - m) : g - (g - m) * (1.0f - s.one_m_b1);
  v = v * s.b2;
  v = v + s.one_m_b2 * (g * g);
  const float denom = sqrtf(v) / s.bc2_sqrt + s.eps;
  p = p + s.neg_step_size * (m / denom);
}

// One tensor of a batched AdamW launch: its blocks start at block0.
struct AdamJob {
  float* p;
  const float* g;
  float* m;
  float* v;
  bf16_t* shadow;  // optional bf16 copy of the updated p
  int64_t n;
  int64_t block0;
};
constexpr int kAdamMaxJobs = 48;        // tensors per launch (the table travels as kernel arguments, 2.7 KB)
constexpr int kAdamPerThread = 8;       // two 16-byte vectors of each stream per thread
constexpr int kAdamPerBlock = 256 * kAdamPerThread;
struct AdamJobs {
  int32_t n;
  AdamJob job[kAdamMaxJobs];
};
static_assert(sizeof(AdamJobs) + sizeof(AdamScalars) <= 4000, "kernel arguments fit the 4 KB limit");

// Every tensor of the table in one launch: a workgroup updates 2048 consecutive elements of one tensor with 16-byte
// loads and stores of p, g, m and v (28 bytes of HBM traffic per element, 30 with the bf16 copy). Tensors start
// 16-byte aligned (checked on the host); a tail shorter than a vector goes element by element.
__global__ __launch_bounds__(256) void adamw_kernel(AdamJobs jobs, AdamScalars s) {
  int j = 0;
  while (j + 1 < jobs.n && (int64_t)blockIdx.x >= jobs.job[j + 1].block0) ++j;
  const AdamJob& J = jobs.job[j];
  const int64_t base = ((int64_t)blockIdx.x - J.block0) * kAdamPerBlock;
#pragma unroll
  for (int u = 0; u < kAdamPerThread / 4; ++u) {
    const int64_t i = base + (int64_t)(u * 256 + threadIdx.x) * 4;
    if (i + 4 <= J.n) {
      f32x4 p = *(const f32x4*)(J.p + i), m = *(const f32x4*)(J.m + i), v = *(const f32x4*)(J.v + i);
      const f32x4 g = *(const f32x4*)(J.g + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float pe = p[e], me = m[e], ve = v[e];
        adam_element(pe, g[e], me, ve, s);
        p[e] = pe;
        m[e] = me;
        v[e] = ve;
      }
      *(f32x4*)(J.p + i) = p;
      *(f32x4*)(J.m + i) = m;
      *(f32x4*)(J.v + i) = v;
      if (J.shadow) *(u32x2*)(J.shadow + i) = u32x2{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
    } else {
      for (int64_t k = i; k < J.n; ++k) {
        float p = J.p[k], m = J.m[k], v = J.v[k];
        adam_element(p, J.g[k], m, v, s);
        J.p[k] = p;
        J.m[k] = m;
        J.v[k] = v;
        if (J.shadow) J.shadow[k] = f32_to_bf16(p);
      }
    }
  }
}

}  // namespace noise

using namespace noise;

extern "C" int noise_fitness(const float* losses, int64_t members, int64_t pairs, float* fitness, float* weight,
                             void* stream) {
  NOISE_REQUIRE(losses && fitness && weight, "NULL pointer argument");
  NOISE_REQUIRE(members >= 2 && members % 2 == 0, "members %lld must be even and >= 2", (long long)members);
  NOISE_REQUIRE(pairs > 0, "pairs must be positive");
  NoiseTimer tm(kTimeFitness, (hipStream_t)stream);
  hipLaunchKernelGGL(fitness_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, losses, members / 2, pairs, fitness,
                     weight);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" int noise_outer_grad(const float* rows, int64_t stride, int64_t a_off, int64_t b_off, const float* weight,
                                int64_t pairs, int64_t out, int64_t in, float scale, int32_t accumulate, float* grad,
                                void* stream) {
  NOISE_REQUIRE(rows && weight && grad, "NULL pointer argument");
  NOISE_REQUIRE(pairs > 0 && in > 0 && a_off >= 0 && stride > 0, "bad sizes");
  if (b_off >= 0)  // a matrix: a one-job launch of the grouped kernel
    return noise_outer_grad_batch(rows, stride, weight, pairs, 1, &a_off, &b_off, &out, &in, &grad, scale, accumulate,
                                  stream);
  NOISE_REQUIRE(a_off + in <= stride, "slice beyond the noise row");
  NoiseTimer tm(kTimeVectorGrad, (hipStream_t)stream);
  hipLaunchKernelGGL(vector_grad_kernel, dim3((unsigned)((in + 7) / 8)), dim3(256), 0, (hipStream_t)stream, rows,
                     stride, a_off, weight, pairs, in, scale, accumulate ? 1 : 0, grad);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" int noise_outer_grad_batch(const float* rows, int64_t stride, const float* weight, int64_t pairs,
                                      int32_t n, const int64_t* a_off, const int64_t* b_off, const int64_t* out,
                                      const int64_t* in, float* const* grads, float scale, int32_t accumulate,
                                      void* stream) {
  NOISE_REQUIRE(rows && weight && a_off && b_off && out && in && grads, "NULL pointer argument");
  NOISE_REQUIRE(pairs > 0 && stride > 0 && n >= 0, "bad sizes");
  for (int32_t j = 0; j < n; ++j) {  // every matrix is checked before anything is launched
    NOISE_REQUIRE(grads[j], "NULL gradient pointer (matrix %d)", j);
    NOISE_REQUIRE(out[j] > 0 && in[j] > 0 && out[j] <= INT32_MAX && in[j] <= INT32_MAX, "matrix %d: bad shape", j);
    NOISE_REQUIRE(a_off[j] >= 0 && b_off[j] >= 0 && a_off[j] + out[j] <= stride && b_off[j] + in[j] <= stride,
                  "matrix %d: slice beyond the noise row", j);
  }
  NoiseTimer tm(kTimeUpdate, (hipStream_t)stream);
  for (int32_t j0 = 0; j0 < n; j0 += kOgMaxJobs) {
    OgJobs jobs;
    memset(&jobs, 0, sizeof(jobs));
    jobs.n = n - j0 < kOgMaxJobs ? n - j0 : kOgMaxJobs;
    jobs.accumulate = accumulate ? 1 : 0;
    int64_t tiles = 0;
    for (int k = 0; k < jobs.n; ++k) {
      const int32_t j = j0 + k;
      OgJob& g = jobs.job[k];
      g.a_off = a_off[j]; g.b_off = b_off[j]; g.out = (int32_t)out[j]; g.in = (int32_t)in[j]; g.grad = grads[j];
      g.n_in_tiles = (int32_t)((in[j] + kOgTile - 1) / kOgTile);
      g.tile0 = (int32_t)tiles;
      tiles += (int64_t)g.n_in_tiles * ((out[j] + kOgTile - 1) / kOgTile);
      NOISE_REQUIRE(tiles <= INT32_MAX, "too many tiles");
    }
    if (tiles == 0) continue;
    NOISE_REQUIRE(tiles + 7 <= INT32_MAX, "too many tiles");
    jobs.total = (int32_t)tiles;
    hipLaunchKernelGGL(outer_grad_kernel, dim3((unsigned)((tiles + 7) / 8 * 8)), dim3(256), 0, (hipStream_t)stream,
                       rows, stride, (const void*)rows, stride, 0, weight, pairs, scale, jobs);
    NOISE_LAUNCH_CHECK();
  }
  return NOISE_OK;
}

// weight_error[o, i] = scale sum_t error[t, o] x[t, i] (train/val/dust.py:386-392, run.py:861-867, the einsum
// 'btd,bti->di'), on the grouped outer-product kernel with one job, the tokens as its K.
extern "C" int noise_reassemble(const float* error, int64_t error_ld, const void* x, int32_t x_bf16, int64_t x_ld,
                                int64_t tokens, int64_t d_out, int64_t d_in, float scale, float* grad, void* stream) {
  NOISE_REQUIRE(error && x && grad, "NULL pointer argument");
  NOISE_REQUIRE(tokens > 0 && d_out > 0 && d_in > 0 && d_out <= INT32_MAX && d_in <= INT32_MAX, "bad sizes");
  NOISE_REQUIRE(error_ld >= d_out && x_ld >= d_in, "row strides shorter than the rows");
  OgJobs jobs;
  memset(&jobs, 0, sizeof(jobs));
  jobs.n = 1;
  OgJob& g = jobs.job[0];
  g.out = (int32_t)d_out; g.in = (int32_t)d_in; g.grad = grad;
  g.n_in_tiles = (int32_t)((d_in + kOgTile - 1) / kOgTile);
  const int64_t tiles = (int64_t)g.n_in_tiles * ((d_out + kOgTile - 1) / kOgTile);
  NOISE_REQUIRE(tiles + 7 <= INT32_MAX, "too many tiles");
  jobs.total = (int32_t)tiles;
  NoiseTimer tm(kTimeReassemble, (hipStream_t)stream);
  hipLaunchKernelGGL(outer_grad_kernel, dim3((unsigned)((tiles + 7) / 8 * 8)), dim3(256), 0, (hipStream_t)stream,
                     error, error_ld, x, x_ld, x_bf16 ? 1 : 0, (const float*)nullptr, tokens, scale, jobs);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

// weight_error[v, :] = sum over the tokens t with ids[t] == v of error[t, :] (the embedding case of reassemble:
// index_add_ over the token ids). One workgroup per table row (and 512 columns) scans the ids 128 at a time: each
// thread tests one id, the two waves' ballots go to LDS, and every thread then adds the matching error rows in
// position order, 4 columns a thread. The order is fixed, so the sums are deterministic. Other ids add nothing.
__global__ __launch_bounds__(128) void scatter_rows_kernel(const float* __restrict__ error, int64_t error_ld,
                                                           const int64_t* __restrict__ ids, int64_t tokens,
                                                           int64_t width, float* __restrict__ grad) {
  __shared__ uint64_t mask[2];
  const int64_t v = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t c0 = (int64_t)blockIdx.y * 512 + tid * 4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t t0 = 0; t0 < tokens; t0 += 128) {
    const int64_t t = t0 + tid;
    const uint64_t b = __ballot(t < tokens && ids[t] == v);
    if ((tid & 63) == 0) mask[tid >> 6] = b;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      uint64_t mk = mask[w];
      while (mk) {
        const int k = __builtin_ctzll(mk);
        mk &= mk - 1;
        const float* row = error + (t0 + 64 * w + k) * error_ld;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c0 + e < width) acc[e] += row[c0 + e];
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (c0 + e < width) grad[v * width + c0 + e] = acc[e];
}

extern "C" int noise_reassemble_embedding(const float* error, int64_t error_ld, const int64_t* ids, int64_t tokens,
                                          int64_t vocab, int64_t width, float* grad, void* stream) {
  NOISE_REQUIRE(error && ids && grad, "NULL pointer argument");
  NOISE_REQUIRE(tokens > 0 && vocab > 0 && width > 0 && error_ld >= width, "bad sizes");
  NOISE_REQUIRE(vocab <= INT32_MAX && (width + 511) / 512 <= 65535, "table too large");
  NoiseTimer tm(kTimeReassemble, (hipStream_t)stream);
  hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)vocab, (unsigned)((width + 511) / 512)), dim3(128), 0,
                     (hipStream_t)stream, error, error_ld, ids, tokens, width, grad);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

static AdamScalars adam_scalars(float lr, float beta1, float beta2, float eps, float weight_decay, int64_t step) {
  // host scalars in double, as torch's optimizer forms them from Python floats
  const double bc1 = 1.0 - pow((double)beta1, (double)step);
  const double bc2 = 1.0 - pow((double)beta2, (double)step);
  AdamScalars s;
  s.lr_wd = (float)(1.0 - (double)lr * (double)weight_decay);
  s.one_m_b1 = (float)(1.0 - (double)beta1);
  s.b2 = beta2;
  s.one_m_b2 = (float)(1.0 - (double)beta2);
  s.neg_step_size = (float)(-((double)lr / bc1));
  s.bc2_sqrt = (float)sqrt(bc2);
  s.eps = eps;
  return s;
}

static bool aligned16(const void* q) { return q == nullptr || ((uintptr_t)q & 15) == 0; }

extern "C" int noise_adamw_batch(int32_t n, float* const* p, const float* const* g, float* const* m, float* const* v,
                                 uint16_t* const* shadow, const int64_t* numel, float lr, float beta1, float beta2,
                                 float eps, float weight_decay, int64_t step, void* stream) {
  NOISE_REQUIRE(n >= 0 && (n == 0 || (p && g && m && v && numel)), "NULL pointer argument");
  NOISE_REQUIRE(step >= 1, "step >= 1 required");
  for (int32_t j = 0; j < n; ++j) {
    NOISE_REQUIRE(numel[j] >= 0, "tensor %d: negative size", j);
    if (numel[j] == 0) continue;
    NOISE_REQUIRE(p[j] && g[j] && m[j] && v[j], "tensor %d: NULL pointer", j);
    NOISE_REQUIRE(aligned16(p[j]) && aligned16(g[j]) && aligned16(m[j]) && aligned16(v[j]) &&
                      (!shadow || ((uintptr_t)shadow[j] & 7) == 0),
                  "tensor %d: p, g, m, v must be 16-byte aligned (the bf16 copy 8-byte aligned)", j);
  }
  const AdamScalars s = adam_scalars(lr, beta1, beta2, eps, weight_decay, step);
  NoiseTimer tm(kTimeAdamw, (hipStream_t)stream);
  // One cursor over the tensors: each launch takes the next kAdamMaxJobs non-empty ones, so an empty tensor never
  // shifts a tensor into two launches.
  for (int32_t j = 0; j < n;) {
    AdamJobs jobs;
    memset(&jobs, 0, sizeof(jobs));
    int64_t blocks = 0;
    for (; j < n && jobs.n < kAdamMaxJobs; ++j) {
      if (numel[j] == 0) continue;
      AdamJob& J = jobs.job[jobs.n++];
      J.p = p[j]; J.g = g[j]; J.m = m[j]; J.v = v[j]; J.shadow = shadow ? (bf16_t*)shadow[j] : nullptr;
      J.n = numel[j];
      J.block0 = blocks;
      blocks += (numel[j] + kAdamPerBlock - 1) / kAdamPerBlock;
    }
    if (blocks == 0) continue;
    NOISE_REQUIRE(blocks <= INT32_MAX, "too many elements");
    hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, jobs, s);
    NOISE_LAUNCH_CHECK();
  }
  return NOISE_OK;
}

extern "C" int noise_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                           float eps, float weight_decay, int64_t step, uint16_t* shadow, void* stream) {
  NOISE_REQUIRE(p && g && m && v, "NULL pointer argument");
  NOISE_REQUIRE(n >= 0 && step >= 1, "n >= 0 and step >= 1 required");
  return noise_adamw_batch(1, &p, &g, &m, &v, shadow ? &shadow : nullptr, &n, lr, beta1, beta2, eps, weight_decay,
                           step, stream);
}
