// Stand-alone entry points over the shared kernels: the windowed attention forward, the two credit passes and the
// perturbed linear of one layer.
#include <string.h>

#include "gemm.h"
#include "window_flash.h"

namespace noise {

// y = acc + s_m u[row] a_m[col] for the rows' member m; optional fp32 store; per-row partial sums of y^2 over the
// 256-column tile (part[row, n_tile]).
struct EpiLowrank {
  int T;
  const float* noise;
  int64_t stride, a_off;
  const float* sign;
  const float* u;     // [M] x . b of each row
  float* y;           // [M, N] or NULL
  int64_t ldy;
  float* part;        // [M, n_tiles] or NULL
  int n_tiles;
  static constexpr int kRows = kEpiRows;
  struct Wave {
    int row_base;
    float k;  // the lane's row's s_m u[row]
    f32x4 a;
  };
  struct Pre {};
  __device__ __forceinline__ void begin(int row_base, int n0, int lane, int nrows, Wave& w) const {
    const int m = row_base / T;
    w.row_base = row_base;
    w.a = *(const f32x4*)(noise + (int64_t)m * stride + a_off + n0 + 4 * lane);
    w.k = lane < nrows ? sign[m] * u[row_base + lane] : 0.f;
  }
  __device__ __forceinline__ void load(int, int, int, const Wave&, Pre&) const {}
  template <int R>
  __device__ __forceinline__ void rows(int row0, int n0, int n_tile, int lane, const Wave& w, const Pre&,
                                       f32x4 (&v)[R]) const {
    static_assert(R == 8, "warp_sum8 reduces 8 rows");
    float ss[R];
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const float k = lane_val(w.k, row0 - w.row_base + q);
      ss[q] = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[q][e] += k * w.a[e];
        ss[q] += v[q][e] * v[q][e];
      }
      if (y) *(f32x4*)(y + (int64_t)(row0 + q) * ldy + n0 + 4 * lane) = v[q];
    }
    if (part) {
      const float tot = warp_sum8(ss, lane);
      if ((lane & 7) == 0) part[(int64_t)(row0 + (lane >> 3)) * n_tiles + n_tile] = tot;
    }
  }
};

// u[r] = x[r % xrows] . b_{r / T}
__global__ __launch_bounds__(256) void lowrank_u_kernel(const bf16_t* __restrict__ x, int64_t xrows, int K, int T,
                                                        const float* __restrict__ noise, int64_t stride, int64_t b_off,
                                                        float* __restrict__ u, int64_t M) {
  const int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= M) return;
  const int lane = threadIdx.x & 63;
  const float* bv = noise + (r / T) * stride + b_off;
  const bf16_t* xr = x + (r % xrows) * K;
  float d = 0.f;
  for (int c = lane; c < K; c += 64) d += bf16_to_f32(xr[c]) * bv[c];
  d = warp_sum(d);
  if (lane == 0) u[r] = d;
}

// sumsq[m] = sum of the member's per-row partials: one workgroup per member, fixed order (deterministic).
__global__ __launch_bounds__(256) void member_part_sum_kernel(const float* __restrict__ part, int per_member,
                                                              float* __restrict__ out) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  float s = 0.f;
  for (int i = threadIdx.x; i < per_member; i += 256) s += part[(int64_t)m * per_member + i];
  s = warp_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[m] = (red[0] + red[1]) + (red[2] + red[3]);
}

using LTile = GemmShape<256, 256, 32, 2, 2>;

}  // namespace noise

using namespace noise;

extern "C" int noise_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t batch, int32_t heads,
                               int64_t T, int64_t stride_b, int64_t stride_t, int32_t window, uint16_t* out,
                               int64_t out_stride_b, int64_t out_stride_t, float* lse, void* stream) {
  NOISE_REQUIRE(q && k && v && out, "NULL pointer argument");
  NOISE_REQUIRE(batch > 0 && batch <= 65535 && heads > 0 && heads <= 65535, "batch / heads outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  NOISE_REQUIRE(stride_t % 8 == 0 && stride_b % 8 == 0 && out_stride_t % 4 == 0, "strides must keep 16-byte rows");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = q; a.y = k; a.v = v;
  a.x_sb = a.y_sb = a.v_sb = stride_b;
  a.x_st = a.y_st = a.v_st = stride_t;
  a.out = out; a.o_sb = out_stride_b; a.o_st = out_stride_t;
  a.lse_out = lse;
  a.heads = heads; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeAttention, (hipStream_t)stream);
  NOISE_CHECK_HIP((launch_flash<kAttn, false, 1>(a, batch, heads, (hipStream_t)stream)));
  return NOISE_OK;
}

extern "C" int noise_credit_lse(const uint16_t* q, const uint16_t* k, int64_t rows, int64_t T, int32_t window,
                                float* lse, void* stream) {
  NOISE_REQUIRE(q && k && lse, "NULL pointer argument");
  NOISE_REQUIRE(rows > 0 && rows <= 65535, "rows outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = q; a.y = k;
  a.x_sb = a.y_sb = T * 64; a.x_st = a.y_st = 64;
  a.lse_out = lse;
  a.heads = 1; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeCreditLse, (hipStream_t)stream);
  NOISE_CHECK_HIP((launch_flash<kLse, false, 1>(a, rows, 1, (hipStream_t)stream)));
  return NOISE_OK;
}

extern "C" int noise_credit_key_context(const uint16_t* q, const uint16_t* k, const uint16_t* values,
                                        const uint16_t* hub, int64_t rows, int64_t T, int32_t window, float* lse,
                                        float* center, void* stream) {
  NOISE_REQUIRE(q && k && values && hub && lse && center, "NULL pointer argument");
  NOISE_REQUIRE(rows > 0 && rows <= 65535, "rows outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = q; a.y = k; a.v = values; a.hub = hub;
  a.x_sb = a.y_sb = a.v_sb = T * 64; a.x_st = a.y_st = a.v_st = 64;
  a.lse_out = lse; a.center_out = center;
  a.heads = 1; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeCreditCenter, (hipStream_t)stream);
  NOISE_CHECK_HIP((launch_flash<kCenter, false, 1>(a, rows, 1, (hipStream_t)stream)));
  return NOISE_OK;
}

extern "C" int noise_credit_value(const uint16_t* q, const uint16_t* k, const float* lse, const float* src, int64_t rows,
                                  int64_t T, int32_t window, int32_t hi_lo, float* out, void* stream) {
  NOISE_REQUIRE(q && k && lse && src && out, "NULL pointer argument");
  NOISE_REQUIRE(rows > 0 && rows <= 65535, "rows outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(window >= 0, "negative window");
  FlashArgs a;
  memset(&a, 0, sizeof(a));
  a.x = k; a.y = q; a.v = src;
  a.x_sb = a.y_sb = a.v_sb = T * 64; a.x_st = a.y_st = a.v_st = 64;
  a.lse_in = lse;
  a.out = out; a.o_sb = T * 64; a.o_st = 64;
  a.heads = 1; a.T = (int)T; a.window = window;
  NoiseTimer tm(kTimeCreditValue, (hipStream_t)stream);
  if (hi_lo)
    NOISE_CHECK_HIP((launch_flash<kCredit, true, 1>(a, rows, 1, (hipStream_t)stream)));
  else
    NOISE_CHECK_HIP((launch_flash<kCredit, false, 1>(a, rows, 1, (hipStream_t)stream)));
  return NOISE_OK;
}

static inline size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

extern "C" size_t noise_lowrank_workspace(int64_t m, int64_t T, int64_t in, int64_t out, int32_t x_shared) {
  (void)in; (void)x_shared;
  const int64_t M = m * T;
  return al256((size_t)M * 4) + al256((size_t)M * (out / LTile::BN) * 4) + (x_shared ? al256((size_t)M * in * 2) : 0);
}

extern "C" int noise_lowrank(const uint16_t* x, int32_t x_shared, const uint16_t* w, const float* noise,
                             int64_t noise_stride, int64_t a_off, int64_t b_off, const float* sign, int64_t m, int64_t T,
                             int64_t in, int64_t out, float* y, float* sumsq, void* workspace, size_t workspace_bytes,
                             void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  NOISE_REQUIRE(x && w && noise && sign, "NULL pointer argument");
  NOISE_REQUIRE(m > 0 && T > 0 && T % LTile::WTM == 0, "T = %lld must be a positive multiple of %d", (long long)T,
                LTile::WTM);
  NOISE_REQUIRE(in > 0 && in % LTile::BK == 0 && out > 0 && out % LTile::BN == 0, "in %% 32 and out %% 256 must be 0");
  const int64_t M = m * T;
  NOISE_REQUIRE(M <= (int64_t)INT32_MAX / 4, "m * T too large");
  NOISE_REQUIRE(workspace && workspace_bytes >= noise_lowrank_workspace(m, T, in, out, x_shared),
                "workspace too small");
  float* u = (float*)workspace;
  float* part = (float*)((char*)workspace + al256((size_t)M * 4));
  const bf16_t* A = (const bf16_t*)x;
  if (x_shared) {  // replicate the shared operand per member (workspace), so the grouped GEMM streams one [M, in] A
    bf16_t* rep = (bf16_t*)((char*)part + al256((size_t)M * (out / LTile::BN) * 4));
    for (int64_t i = 0; i < m; ++i)
      NOISE_CHECK_HIP(hipMemcpyAsync(rep + i * T * in, x, (size_t)T * in * 2, hipMemcpyDeviceToDevice, stream));
    A = rep;
  }
  hipLaunchKernelGGL(lowrank_u_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream, A, M, (int)in, (int)T,
                     noise, noise_stride, b_off, u, M);
  NOISE_LAUNCH_CHECK();
  EpiLowrank epi{(int)T, noise, noise_stride, a_off, sign, u, y, out, sumsq ? part : nullptr, (int)(out / LTile::BN)};
  NOISE_CHECK_HIP((prepare_gemm<LTile, EpiLowrank>()));
  {
    NoiseTimer tm(kTimeLowrank, stream);
    NOISE_CHECK_HIP((launch_gemm<LTile>(A, in, w, in, (int)M, (int)out, (int)in, epi, stream)));
  }
  if (sumsq) {
    hipLaunchKernelGGL(member_part_sum_kernel, dim3((unsigned)m), dim3(256), 0, stream, part,
                       (int)(T * (out / LTile::BN)), sumsq);
    NOISE_LAUNCH_CHECK();
  }
  return NOISE_OK;
}
