// Fitness, gradient assembly and the AdamW step of the EGGROLL update
// (archive/10M/train/val/eggroll.py:151-167; optimizer semantics of torch.optim.AdamW as built at :205).
#include <math.h>

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

// grad[o, i] = scale sum_j w_j a_j[o] b_j[i]: fp32 tiles of 64 x 64 outputs, 4 x 4 per thread, 16 directions per step.
__global__ __launch_bounds__(256) void outer_grad_kernel(const float* __restrict__ rows, int64_t stride, int64_t a_off,
                                                         int64_t b_off, const float* __restrict__ weight, int64_t pairs,
                                                         int64_t out, int64_t in, float scale, float* __restrict__ grad) {
  __shared__ float as[16][64];
  __shared__ float bs[16][64];
  const int o0 = blockIdx.y * 64, i0 = blockIdx.x * 64;
  const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  float acc[4][4] = {};
  for (int64_t j0 = 0; j0 < pairs; j0 += 16) {
    for (int e = tid; e < 16 * 64; e += 256) {
      const int jj = e / 64, c = e % 64;
      const int64_t j = j0 + jj;
      float av = 0.f, bv = 0.f;
      if (j < pairs) {
        const float* row = rows + j * stride;
        av = (o0 + c < out) ? row[a_off + o0 + c] : 0.f;
        bv = (i0 + c < in) ? weight[j] * row[b_off + i0 + c] : 0.f;
      }
      as[jj][c] = av;
      bs[jj][c] = bv;
    }
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      float a4[4], b4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) { a4[u] = as[jj][ty * 4 + u]; b4[u] = bs[jj][tx * 4 + u]; }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[u][v] += a4[u] * b4[v];
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t o = o0 + ty * 4 + u, i = i0 + tx * 4 + v;
      if (o < out && i < in) grad[o * in + i] = scale * acc[u][v];
    }
}

// grad[i] = scale sum_j w_j eps_j[i] (1-D parameters: eggroll.py:163)
__global__ void vector_grad_kernel(const float* __restrict__ rows, int64_t stride, int64_t a_off,
                                   const float* __restrict__ weight, int64_t pairs, int64_t n, float scale,
                                   float* __restrict__ grad) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int64_t j = 0; j < pairs; ++j) s += weight[j] * rows[j * stride + a_off + i];
  grad[i] = scale * s;
}

struct AdamScalars {
  float lr_wd;       // 1 - lr * weight_decay
  float one_m_b1;    // lerp weight
  float b2, one_m_b2;
  float neg_step_size;  // -lr / (1 - b1^step)
  float bc2_sqrt;       // sqrt(1 - b2^step)
  float eps;
};

// torch.optim.AdamW (foreach path) per element: p *= 1 - lr wd; m = lerp(m, g, 1 - b1); v = v b2 + (1 - b2) g g;
// p += -step_size * m / (sqrt(v) / bc2_sqrt + eps).
__global__ void adamw_kernel(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                             float* __restrict__ v, int64_t n, AdamScalars s, bf16_t* __restrict__ shadow) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float gi = g[i];
  float pi = p[i] * s.lr_wd;
  float mi = m[i];
  // torch's lerp: weight < 0.5 ? start + w (end - start) : end - (end - start) (1 - w)
  mi = (s.one_m_b1 < 0.5f) ? mi + s.one_m_b1 * (gi - mi) : gi - (gi - mi) * (1.0f - s.one_m_b1);
  float vi = v[i] * s.b2;
  vi = vi + s.one_m_b2 * (gi * gi);
  const float denom = sqrtf(vi) / s.bc2_sqrt + s.eps;
  pi = pi + s.neg_step_size * (mi / denom);
  p[i] = pi;
  m[i] = mi;
  v[i] = vi;
  if (shadow) shadow[i] = f32_to_bf16(pi);
}

}  // namespace noise

using namespace noise;

extern "C" int noise_fitness(const float* losses, int64_t members, int64_t pairs, float* fitness, float* weight,
                             void* stream) {
  NOISE_REQUIRE(losses && fitness && weight, "NULL pointer argument");
  NOISE_REQUIRE(members >= 2 && members % 2 == 0, "members %lld must be even and >= 2", (long long)members);
  NOISE_REQUIRE(pairs > 0, "pairs must be positive");
  hipLaunchKernelGGL(fitness_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, losses, members / 2, pairs, fitness,
                     weight);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" int noise_outer_grad(const float* rows, int64_t stride, int64_t a_off, int64_t b_off, const float* weight,
                                int64_t pairs, int64_t out, int64_t in, float scale, float* grad, void* stream) {
  NOISE_REQUIRE(rows && weight && grad, "NULL pointer argument");
  NOISE_REQUIRE(pairs > 0 && in > 0 && a_off >= 0 && stride > 0, "bad sizes");
  NoiseTimer tm(kTimeUpdate, (hipStream_t)stream);
  if (b_off < 0) {
    NOISE_REQUIRE(a_off + in <= stride, "slice beyond the noise row");
    hipLaunchKernelGGL(vector_grad_kernel, dim3((unsigned)((in + 255) / 256)), dim3(256), 0, (hipStream_t)stream, rows,
                       stride, a_off, weight, pairs, in, scale, grad);
  } else {
    NOISE_REQUIRE(out > 0 && a_off + out <= stride && b_off + in <= stride, "slice beyond the noise row");
    dim3 grid((unsigned)((in + 63) / 64), (unsigned)((out + 63) / 64));
    hipLaunchKernelGGL(outer_grad_kernel, grid, dim3(256), 0, (hipStream_t)stream, rows, stride, a_off, b_off, weight,
                       pairs, out, in, scale, grad);
  }
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" int noise_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                           float eps, float weight_decay, int64_t step, uint16_t* shadow, void* stream) {
  NOISE_REQUIRE(p && g && m && v, "NULL pointer argument");
  NOISE_REQUIRE(n >= 0 && step >= 1, "n >= 0 and step >= 1 required");
  if (n == 0) return NOISE_OK;
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
  hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, p, g, m, v, n,
                     s, shadow);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}
