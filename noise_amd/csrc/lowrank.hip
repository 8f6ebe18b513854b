// The perturbed linear of EGGROLL, y_i = x W^T + s_i (x . b_i) a_i^T (archive/10M/train/val/eggroll.py:56-58), as a
// library entry point, in the reference's bf16 autocast arithmetic: the matmul output x W^T and the dot x . b_i are
// rounded to bf16 (b_i and a_i enter as bf16), and the rank-1 term is added in fp32.
//
//  * Per-member x ([m, T, in]): one grouped GEMM over the m T rows, the rank-1 term in its epilogue.
//  * Shared x ([T, in], config 2's single perturbed linear): X W^T is computed once per 256 x 256 tile
//    and every member's rank-1 term and sum of squares S_i = sum_{r,c} y_i[r, c]^2 come out of that one accumulator
//    tile, in registers. Two evaluations of S_i:
//      - per element: y = c + (s_i u_i[r]) a_i[c] and y^2 summed for every member (fp32 VALU, 2 FMAs per element and
//        member; the only form that can also store y);
//      - by the expansion S_i = sum c^2 + 2 s_i sum_c a_i[c] E_i[c] + s_i^2 (sum_r u_i[r]^2)(sum_c a_i[c]^2), with
//        E_i[c] = sum_r u_i[r] c[r, c] taken on the MFMA units straight from the accumulator registers (the
//        accumulator layout of v_mfma_f32_32x32x16_bf16 is the B operand of the next product with the rows as k), so
//        the per-member work costs 1/8 of the tile's main loop instead of 64 VALU passes over the tile.
//    Both use the same rounded c, u and a; they differ only in the fp32 summation order.
#include <string.h>

#include <mutex>

#include "gemm.h"

namespace noise {

// ---- per-member x ---------------------------------------------------------------------------------------------

// y = c + k a_m[col] for the rows' member m (k = s_m u[row]); optional fp32 store; per-row partial sums of y^2 over
// the 256-column tile (part[row, n_tile]).
struct EpiLowrank {
  int T;
  const float* noise;
  int64_t stride, a_off;
  const float* sign;
  const float* u;     // [M] bf16-rounded x . b of each row
  float* y;           // [M, N] or NULL
  int64_t ldy;
  float* part;        // [M, n_tiles] or NULL
  int n_tiles;
  static constexpr int kRows = kEpiRows;
  struct Wave {
    int row_base;
    float k;  // the lane's row's s_m u[row]
    f32x4 a;  // bf16-rounded a_m at the lane's 4 columns
  };
  struct Pre {};
  __device__ __forceinline__ void begin(int row_base, int n0, int lane, int nrows, Wave& w) const {
    const int m = row_base / T;
    w.row_base = row_base;
    const f32x4 a = *(const f32x4*)(noise + (int64_t)m * stride + a_off + n0 + 4 * lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) w.a[e] = bf16_to_f32(f32_to_bf16(a[e]));
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

// u[r] = bf16(x[r] . bf16(b_{r / T})), one wave per row.
__global__ __launch_bounds__(256) void lowrank_dot_kernel(const bf16_t* __restrict__ x, int K, int T,
                                                          const float* __restrict__ noise, int64_t stride,
                                                          int64_t b_off, float* __restrict__ u, int64_t M) {
  const int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= M) return;
  const int lane = threadIdx.x & 63;
  const float* bv = noise + (r / T) * stride + b_off;
  const bf16_t* xr = x + r * K;
  float d = 0.f;
  for (int c = lane; c < K; c += 64) d += bf16_to_f32(xr[c]) * bf16_to_f32(f32_to_bf16(bv[c]));
  d = warp_sum(d);
  if (lane == 0) u[r] = bf16_to_f32(f32_to_bf16(d));
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

// ---- shared x ---------------------------------------------------------------------------------------------------

constexpr int kMemberTile = 32;  // members per MFMA tile (the N of v_mfma_f32_32x32x16_bf16)
constexpr int kURows = 128;      // rows per workgroup of shared_u_kernel (4 waves of 32)

// Per member (mp workgroups; members m .. mp - 1 are zero padding): bt = bf16(b_i) [mp, in]; the bf16-rounded a_i as
// fp32 both member-major (am [mp, out]) and column-major (at [out, mp]); asq[i] = sum_c a_i[c]^2.
__global__ __launch_bounds__(256) void shared_prep_kernel(const float* __restrict__ noise, int64_t stride,
                                                          int64_t a_off, int64_t b_off, int m, int mp, int in, int out,
                                                          bf16_t* __restrict__ bt, float* __restrict__ am,
                                                          float* __restrict__ at, float* __restrict__ asq) {
  __shared__ float red[4];
  const int i = blockIdx.x;
  const bool live = i < m;
  const float* a = live ? noise + (int64_t)i * stride + a_off : nullptr;
  const float* b = live ? noise + (int64_t)i * stride + b_off : nullptr;
  float s = 0.f;
  for (int c = threadIdx.x; c < out; c += 256) {
    const float v = live ? bf16_to_f32(f32_to_bf16(a[c])) : 0.f;
    am[(int64_t)i * out + c] = v;
    at[(int64_t)c * mp + i] = v;
    s = fmaf(v, v, s);
  }
  for (int c = threadIdx.x; c < in; c += 256) bt[(int64_t)i * in + c] = live ? f32_to_bf16(b[c]) : (bf16_t)0;
  s = warp_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) asq[i] = (red[0] + red[1]) + (red[2] + red[3]);
}

// u[i, r] = bf16(x[r] . bt[i]) for every (padded) member i and row r (bf16 [mp, T]), and usq[blk, i] = sum of u[i, r]^2
// over the workgroup's 128 rows. A wave computes 32 rows x one member tile at a time with v_mfma_f32_32x32x16_bf16,
// its operands straight from memory: lane l reads row (or member) l % 32 at k = 8 (l / 32) .. of each 16-deep step.
__global__ __launch_bounds__(256) void shared_u_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ bt,
                                                       int T, int in, int mp, bf16_t* __restrict__ u,
                                                       float* __restrict__ usq) {
  __shared__ float red[4][kMemberTile];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int r0 = blockIdx.x * kURows + wave * 32;
  const bf16_t* xr = x + (int64_t)(r0 + l32) * in + 8 * g;
  for (int mt = 0; mt < mp / kMemberTile; ++mt) {
    const bf16_t* br = bt + (int64_t)(mt * kMemberTile + l32) * in + 8 * g;
    f32x16 e = {};
    for (int k = 0; k < in; k += 32) {  // in % 32 == 0
      e = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8*)(xr + k), *(const bf16x8*)(br + k), e, 0, 0, 0);
      e = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8*)(xr + k + 16), *(const bf16x8*)(br + k + 16), e, 0,
                                                  0, 0);
    }
    // register r: row r0 + (r / 4) 8 + 4 g + r % 4, member mt 32 + l32
    bf16_t* ur = u + (int64_t)(mt * kMemberTile + l32) * T + r0 + 4 * g;
    float sq = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t p0 = pack_bf16x2(e[4 * q], e[4 * q + 1]), p1 = pack_bf16x2(e[4 * q + 2], e[4 * q + 3]);
      *(u32x2*)(ur + 8 * q) = u32x2{p0, p1};
      sq = fmaf(bf16_lo(p0), bf16_lo(p0), sq);
      sq = fmaf(bf16_hi(p0), bf16_hi(p0), sq);
      sq = fmaf(bf16_lo(p1), bf16_lo(p1), sq);
      sq = fmaf(bf16_hi(p1), bf16_hi(p1), sq);
    }
    sq += lane_xor32(sq, lane);  // lanes l and l ^ 32 hold the same member's two halves of the 32 rows
    if (g == 0) red[wave][l32] = sq;
    __syncthreads();
    if (threadIdx.x < kMemberTile) {
      const int t = threadIdx.x;
      usq[(int64_t)blockIdx.x * mp + mt * kMemberTile + t] = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
    }
    __syncthreads();
  }
}

// The 256 x 256 tile of 4 waves of 128 x 128 that both shared-x epilogues take: 64-deep K steps in two LDS stages
// when `in` allows (config 2, alternating builds on one box: the expansion kernel 0.100 against 0.102 ms, the
// per-element one 0.513 against 0.524), 32-deep steps in four otherwise.
using LTile = GemmShape<256, 256, 32, 2, 2>;
using LTile64 = GemmShape<256, 256, 64, 2, 2, 2>;

template <class Epi>
static hipError_t launch_shared_gemm(const uint16_t* x, const uint16_t* w, int64_t T, int64_t in, int64_t out,
                                     const Epi& epi, hipStream_t stream) {
  if (in % LTile64::BK == 0) {
    const hipError_t e = prepare_gemm<LTile64, Epi>();
    if (e != hipSuccess) return e;
    return launch_gemm<LTile64>((const bf16_t*)x, in, (const bf16_t*)w, in, (int)T, (int)out, (int)in, epi, stream);
  }
  const hipError_t e = prepare_gemm<LTile, Epi>();
  if (e != hipSuccess) return e;
  return launch_gemm<LTile>((const bf16_t*)x, in, (const bf16_t*)w, in, (int)T, (int)out, (int)in, epi, stream);
}

// The expansion: per tile, c2[tile] = sum of c^2 over the rounded tile, and cross[tile, i] = sum_c a_i[c] E_i[c] with
// E_i[c] = sum_r u_i[r] c[r, c] over the tile's rows.
struct EpiSharedExpansion {
  static constexpr bool kAccEpilogue = true;
  const bf16_t* u;  // [mp, T]
  const float* at;  // [out, mp] bf16-rounded a, column-major
  float* c2;        // [tiles]
  float* cross;     // [tiles, mp]
  int T, mp;

  template <class S>
  __device__ __forceinline__ void acc_epilogue(f32x16 (&acc)[S::TM][S::TN], unsigned char* smem, int m0, int n0,
                                               int m_tile, int n_tile, int wave, int wm, int wn, int lane) const {
    static_assert(S::TM == 4 && S::TN == 4 && S::kWaves == 4, "a 256 x 256 tile of 4 waves of 128 x 128");
    constexpr int kLd = 17;  // padded lane stride of the partials in LDS
    float* red = (float*)smem;                    // [4 waves][64 lanes][kLd]
    float* red_c2 = red + S::kWaves * 64 * kLd;   // [4 waves]
    const int g = lane >> 5, l32 = lane & 31;
    const int tile = m_tile * gridDim.x + n_tile;
    const int row_w = m0 + wm * S::WTM, col_w = n0 + wn * S::WTN;

    // The tile rounded to bf16 (the autocast matmul output) and packed as B operands with k = rows: register
    // 8 h + e of accumulator (i, j) holds row 16 h + 8 (e / 4) + 4 g + e % 4 of row tile i, column l32 of column
    // tile j, which is k-slot 8 g + e of a 16-deep product over the 16 rows 16 h .. 16 h + 15.
    bf16x8 cb[S::TM][S::TN][2];
    float sq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < S::TM; ++i)
#pragma unroll
      for (int j = 0; j < S::TN; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int e = 0; e < 8; ++e) cb[i][j][h][e] = (__bf16)acc[i][j][8 * h + e];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float c = (float)cb[i][j][h][e];
            sq[e & 3] = fmaf(c, c, sq[e & 3]);
          }
        }
    const float sq_tot = warp_sum((sq[0] + sq[1]) + (sq[2] + sq[3]));
    if (lane == 0) red_c2[wave] = sq_tot;

    for (int mt = 0; mt < mp / kMemberTile; ++mt) {
      // E[j] (members x columns of column tile j) = U (members x rows) . C (rows x columns); the A operand's k-slots
      // follow the rows of cb: elements 0..3 are rows 16 h + 4 g .. +3, elements 4..7 rows 16 h + 8 + 4 g .. +3.
      f32x16 e[S::TN];
#pragma unroll
      for (int j = 0; j < S::TN; ++j) e[j] = f32x16{};
      const bf16_t* ub = u + (int64_t)(mt * kMemberTile + l32) * T + row_w + 4 * g;
#pragma unroll
      for (int i = 0; i < S::TM; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const v4s lo = *(const v4s*)(ub + 32 * i + 16 * h), hi = *(const v4s*)(ub + 32 * i + 16 * h + 8);
          const bf16x8 av = __builtin_bit_cast(bf16x8, s16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
#pragma unroll
          for (int j = 0; j < S::TN; ++j) e[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, cb[i][j][h], e[j], 0, 0, 0);
        }
      // register r of e[j]: member mt 32 + (r / 4) 8 + 4 g + r % 4, column col_w + 32 j + l32
      float cr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) cr[r] = 0.f;
#pragma unroll
      for (int j = 0; j < S::TN; ++j) {
        const float* ap = at + (int64_t)(col_w + 32 * j + l32) * mp + mt * kMemberTile + 4 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 a4 = *(const f32x4*)(ap + 8 * q);
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) cr[4 * q + e4] = fmaf(a4[e4], e[j][4 * q + e4], cr[4 * q + e4]);
        }
      }
      __syncthreads();  // the previous member tile's partials have been read
#pragma unroll
      for (int r = 0; r < 16; ++r) red[(wave * 64 + lane) * kLd + r] = cr[r];
      __syncthreads();
      // thread t: member ml = t / 8 of the tile, part p = t % 8 (lanes 4 p .. 4 p + 3 of its half in every wave)
      const int t = threadIdx.x, ml = t >> 3, p = t & 7;
      const int gg = (ml >> 2) & 1, rr = (ml >> 3) * 4 + (ml & 3);
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < S::kWaves; ++w)
#pragma unroll
        for (int q = 0; q < 4; ++q) s += red[(w * 64 + gg * 32 + 4 * p + q) * kLd + rr];
      s = group_sum8(s);
      if (p == 0) cross[(int64_t)tile * mp + mt * kMemberTile + ml] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) c2[tile] = (red_c2[0] + red_c2[1]) + (red_c2[2] + red_c2[3]);
  }
};

// Per element: y = c + k_i[r] a_i[c] with k_i = s_i u_i (fp32), ss[tile, i] = sum of y^2 over the tile; optional y
// store [m, T, out]. Members go in chunks of 64, whose k values are staged in LDS ([64][256 rows] fp32).
template <bool kStoreY>
struct EpiSharedDirect {
  static constexpr bool kAccEpilogue = true;
  const bf16_t* u;     // [mp, T]
  const float* am;     // [mp, out] bf16-rounded a, member-major
  const float* sign;   // [m]
  float* ss;           // [tiles, m]
  float* y;            // [m, T, out] when kStoreY
  int T, m, out;

  template <class S>
  __device__ __forceinline__ void acc_epilogue(f32x16 (&acc)[S::TM][S::TN], unsigned char* smem, int m0, int n0,
                                               int m_tile, int n_tile, int wave, int wm, int wn, int lane) const {
    static_assert(S::TM == 4 && S::TN == 4 && S::kWaves == 4 && S::BM == 256, "a 256 x 256 tile of 4 waves");
    constexpr int kChunk = 64;
    float* ks = (float*)smem;                // [kChunk][256]
    float* red = ks + kChunk * S::BM;        // [4 waves][kChunk]
    const int g = lane >> 5, l32 = lane & 31;
    const int tile = m_tile * gridDim.x + n_tile;
    const int row_w = m0 + wm * S::WTM, col_w = n0 + wn * S::WTN;
#pragma unroll
    for (int i = 0; i < S::TM; ++i)
#pragma unroll
      for (int j = 0; j < S::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = bf16_to_f32(f32_to_bf16(acc[i][j][r]));

    for (int c0 = 0; c0 < m; c0 += kChunk) {
      const int nm = min(kChunk, m - c0);
      __syncthreads();  // the previous chunk's k values and partials have been read
      for (int idx = threadIdx.x; idx < nm * S::BM; idx += S::kThreads) {
        const int i = idx / S::BM, r = idx % S::BM;
        ks[idx] = sign[c0 + i] * bf16_to_f32(u[(int64_t)(c0 + i) * T + m0 + r]);
      }
      __syncthreads();
#pragma unroll 1
      for (int i = 0; i < nm; ++i) {
        const float* ap = am + (int64_t)(c0 + i) * out + col_w + l32;
        float a[S::TN];
#pragma unroll
        for (int j = 0; j < S::TN; ++j) a[j] = ap[32 * j];
        const float* kp = ks + i * S::BM + wm * S::WTM + 4 * g;
        float s[8];
#pragma unroll
        for (int z = 0; z < 8; ++z) s[z] = 0.f;
#pragma unroll
        for (int it = 0; it < S::TM; ++it)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 k4 = *(const f32x4*)(kp + 32 * it + 8 * q);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
              for (int j = 0; j < S::TN; ++j) {
                const float yv = fmaf(k4[e], a[j], acc[it][j][4 * q + e]);
                s[(e & 1) * 4 + j] = fmaf(yv, yv, s[(e & 1) * 4 + j]);
                if constexpr (kStoreY)
                  y[((int64_t)(c0 + i) * T + row_w + 32 * it + 8 * q + 4 * g + e) * out + col_w + 32 * j + l32] = yv;
              }
          }
        const float tot = warp_sum(((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7])));
        if (lane == 0) red[wave * kChunk + i] = tot;
      }
      __syncthreads();
      if (threadIdx.x < nm) {
        const int t = threadIdx.x;
        ss[(int64_t)tile * m + c0 + t] =
            (red[t] + red[kChunk + t]) + (red[2 * kChunk + t] + red[3 * kChunk + t]);
      }
    }
  }
};

// sumsq[i], one workgroup per member, fixed summation order. Expansion: sum_t c2[t] + 2 s_i sum_t cross[t, i] +
// s_i^2 (sum_b usq[b, i]) asq[i], combined in double. Per element: sum_t ss[t, i].
__global__ __launch_bounds__(256) void shared_finish_kernel(const float* __restrict__ c2,
                                                            const float* __restrict__ cross,
                                                            const float* __restrict__ usq,
                                                            const float* __restrict__ asq,
                                                            const float* __restrict__ ss,
                                                            const float* __restrict__ sign, int tiles, int ublocks,
                                                            int mp, int m, float* __restrict__ sumsq) {
  __shared__ float red[3][4];
  const int i = blockIdx.x, t = threadIdx.x, w = t >> 6;
  float a = 0.f, b = 0.f, c = 0.f;
  if (ss) {
    for (int k = t; k < tiles; k += 256) a += ss[(int64_t)k * m + i];
  } else {
    for (int k = t; k < tiles; k += 256) {
      a += c2[k];
      b += cross[(int64_t)k * mp + i];
    }
    for (int k = t; k < ublocks; k += 256) c += usq[(int64_t)k * mp + i];
  }
  a = warp_sum(a);
  b = warp_sum(b);
  c = warp_sum(c);
  if ((t & 63) == 0) {
    red[0][w] = a;
    red[1][w] = b;
    red[2][w] = c;
  }
  __syncthreads();
  if (t == 0) {
    const float ta = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    if (ss) {
      sumsq[i] = ta;
    } else {
      const double s = sign[i];
      const double tb = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
      const double tc = (red[2][0] + red[2][1]) + (red[2][2] + red[2][3]);
      sumsq[i] = (float)((double)ta + 2.0 * s * tb + s * s * tc * (double)asq[i]);
    }
  }
}

}  // namespace noise

using namespace noise;

static inline size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

namespace {

// Workspace of the shared-x path, carved in this order.
struct SharedWs {
  bf16_t* u;    // [mp, T]
  bf16_t* bt;   // [mp, in]
  float* am;    // [mp, out]
  float* at;    // [out, mp]
  float* asq;   // [mp]
  float* usq;   // [T / 128, mp]
  float* c2;    // [tiles]
  float* part;  // [tiles, mp] (cross or ss)
  size_t bytes;
};

SharedWs shared_ws(void* base, int64_t m, int64_t T, int64_t in, int64_t out) {
  const int64_t mp = (m + kMemberTile - 1) / kMemberTile * kMemberTile;
  const int64_t tiles = (T / LTile::BM) * (out / LTile::BN);
  const size_t sz[8] = {al256((size_t)mp * T * 2),     al256((size_t)mp * in * 2),
                        al256((size_t)mp * out * 4),   al256((size_t)mp * out * 4),
                        al256((size_t)mp * 4),         al256((size_t)(T / kURows) * mp * 4),
                        al256((size_t)tiles * 4),      al256((size_t)tiles * mp * 4)};
  SharedWs w;
  char* p = (char*)base;
  void* ptrs[8];
  size_t off = 0;
  for (int k = 0; k < 8; ++k) {
    ptrs[k] = p ? p + off : nullptr;
    off += sz[k];
  }
  w.u = (bf16_t*)ptrs[0]; w.bt = (bf16_t*)ptrs[1]; w.am = (float*)ptrs[2]; w.at = (float*)ptrs[3];
  w.asq = (float*)ptrs[4]; w.usq = (float*)ptrs[5]; w.c2 = (float*)ptrs[6]; w.part = (float*)ptrs[7];
  w.bytes = off;
  return w;
}

}  // namespace

namespace noise {

// The perturbed embedding of eggroll.py:61-63: out[i, t, c] = W[idx[t], c] + sign[i] a_i[idx[t]] b_i[c] (fp32;
// W fp32 or bf16). A thread takes 4 channels of one (member, token) row.
__global__ __launch_bounds__(256) void lowrank_embed_kernel(const void* __restrict__ w, int w_bf16, int64_t vocab,
                                                            int d, const float* __restrict__ a, int64_t a_stride,
                                                            const float* __restrict__ b, int64_t b_stride,
                                                            const int64_t* __restrict__ idx, const float* __restrict__ sign,
                                                            int64_t T, float* __restrict__ out) {
  const int quads = d / 4;
  const int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;  // quad within the member's [T, d] block
  if (q >= T * quads) return;
  const int i = blockIdx.y;
  const int64_t t = q / quads;
  const int c = (int)(q % quads) * 4;
  const int64_t tok = idx[t];
  float* o = out + ((int64_t)i * T + t) * d + c;
  if (tok < 0 || tok >= vocab) {  // an id outside the table has no row (torch would raise): NaN marks it
    *(f32x4*)o = f32x4{NAN, NAN, NAN, NAN};
    return;
  }
  f32x4 row;
  if (w_bf16) {
    const uint16_t* wr = (const uint16_t*)w + tok * d + c;
#pragma unroll
    for (int e = 0; e < 4; ++e) row[e] = bf16_to_f32(wr[e]);
  } else {
    row = *(const f32x4*)((const float*)w + tok * d + c);
  }
  const float k = sign[i] * a[(int64_t)i * a_stride + tok];
  const f32x4 bv = *(const f32x4*)(b + (int64_t)i * b_stride + c);
  *(f32x4*)o = f32x4{fmaf(k, bv[0], row[0]), fmaf(k, bv[1], row[1]), fmaf(k, bv[2], row[2]), fmaf(k, bv[3], row[3])};
}

}  // namespace noise

extern "C" int noise_lowrank_embed(const void* w, int32_t w_bf16, int64_t vocab, int32_t d, const float* a,
                                   int64_t a_stride, const float* b, int64_t b_stride, const int64_t* idx,
                                   const float* sign, int32_t m, int64_t T, float* out, void* stream) {
  NOISE_REQUIRE(w && a && b && idx && sign && out, "NULL pointer argument");
  NOISE_REQUIRE(m > 0 && m <= 65535 && T > 0 && vocab > 0, "m in [1, 65535], T and vocab positive");
  NOISE_REQUIRE(d > 0 && d % 4 == 0 && b_stride % 4 == 0 && b_stride >= d && a_stride >= vocab,
                "d a positive multiple of 4; b rows 16-byte aligned and at least d long; a rows at least vocab long");
  NOISE_REQUIRE(T * (d / 4) <= (int64_t)INT32_MAX * 256, "T * d too large");
  const int64_t quads = T * (d / 4);
  hipLaunchKernelGGL(lowrank_embed_kernel, dim3((unsigned)((quads + 255) / 256), (unsigned)m), dim3(256), 0,
                     (hipStream_t)stream, w, (int)w_bf16, vocab, (int)d, a, a_stride, b, b_stride, idx, sign, T, out);
  NOISE_LAUNCH_CHECK();
  return NOISE_OK;
}

extern "C" size_t noise_lowrank_workspace(int64_t m, int64_t T, int64_t in, int64_t out, int32_t x_shared) {
  if (m <= 0 || T <= 0 || in <= 0 || out <= 0) return 0;
  if (x_shared) return shared_ws(nullptr, m, T, in, out).bytes;
  const int64_t M = m * T;
  return al256((size_t)M * 4) + al256((size_t)M * (out / LTile::BN) * 4);
}

// Validates the shared-x arguments and launches its kernels on the given workspace (also the body of the
// no-allocation variant).
static int lowrank_shared_run(const uint16_t* x, int32_t mode, const uint16_t* w, const float* noise,
                              int64_t noise_stride, int64_t a_off, int64_t b_off, const float* sign, int64_t m,
                              int64_t T, int64_t in, int64_t out, float* y, float* sumsq, void* workspace,
                              size_t workspace_bytes, hipStream_t stream, bool timed) {
  NOISE_REQUIRE(x && w && noise && sign, "NULL pointer argument");
  NOISE_REQUIRE(mode == 1 || mode == 2, "x_shared must be 0, 1 or 2");
  NOISE_REQUIRE(m > 0 && m <= 65535, "members outside [1, 65535]");
  NOISE_REQUIRE(T > 0 && T % LTile::BM == 0 && T / LTile::BM <= 65535,
                "shared x: T = %lld must be a positive multiple of 256", (long long)T);
  NOISE_REQUIRE(in > 0 && in % LTile::BK == 0 && out > 0 && out % LTile::BN == 0, "in %% 32 and out %% 256 must be 0");
  NOISE_REQUIRE(T * out <= (int64_t)1 << 40 && in <= 65536, "shared x: sizes out of range");
  NOISE_REQUIRE(a_off >= 0 && b_off >= 0 && noise_stride >= a_off + out && noise_stride >= b_off + in,
                "a / b slices outside the noise row");
  const SharedWs ws = shared_ws(workspace, m, T, in, out);
  NOISE_REQUIRE(workspace && workspace_bytes >= ws.bytes, "workspace too small: %zu bytes needed", ws.bytes);
  const int mp = (int)((m + kMemberTile - 1) / kMemberTile * kMemberTile);
  const int tiles = (int)((T / LTile::BM) * (out / LTile::BN));
  const int ublocks = (int)(T / kURows);
  const bool direct = mode == 2 || y != nullptr;
  {
    NoiseTimer tm(timed ? kTimeLowrankPre : -1, stream);
    hipLaunchKernelGGL(shared_prep_kernel, dim3(mp), dim3(256), 0, stream, noise, noise_stride, a_off, b_off, (int)m,
                       mp, (int)in, (int)out, ws.bt, ws.am, ws.at, ws.asq);
    NOISE_LAUNCH_CHECK();
    hipLaunchKernelGGL(shared_u_kernel, dim3(ublocks), dim3(256), 0, stream, (const bf16_t*)x, ws.bt, (int)T, (int)in,
                       mp, ws.u, ws.usq);
    NOISE_LAUNCH_CHECK();
  }
  if (direct) {
    if (y) {
      EpiSharedDirect<true> epi{ws.u, ws.am, sign, ws.part, y, (int)T, (int)m, (int)out};
      NoiseTimer tm(timed ? kTimeLowrank : -1, stream);
      NOISE_CHECK_HIP(launch_shared_gemm(x, w, T, in, out, epi, stream));
    } else {
      EpiSharedDirect<false> epi{ws.u, ws.am, sign, ws.part, nullptr, (int)T, (int)m, (int)out};
      NoiseTimer tm(timed ? kTimeLowrank : -1, stream);
      NOISE_CHECK_HIP(launch_shared_gemm(x, w, T, in, out, epi, stream));
    }
  } else {
    EpiSharedExpansion epi{ws.u, ws.at, ws.c2, ws.part, (int)T, mp};
    NoiseTimer tm(timed ? kTimeLowrank : -1, stream);
    NOISE_CHECK_HIP(launch_shared_gemm(x, w, T, in, out, epi, stream));
  }
  if (sumsq) {
    NoiseTimer tm(timed ? kTimeLowrankPost : -1, stream);
    hipLaunchKernelGGL(shared_finish_kernel, dim3((unsigned)m), dim3(256), 0, stream, ws.c2, ws.part, ws.usq, ws.asq,
                       direct ? ws.part : nullptr, sign, tiles, ublocks, mp, (int)m, sumsq);
    NOISE_LAUNCH_CHECK();
  }
  return NOISE_OK;
}

extern "C" int noise_lowrank(const uint16_t* x, int32_t x_shared, const uint16_t* w, const float* noise,
                             int64_t noise_stride, int64_t a_off, int64_t b_off, const float* sign, int64_t m, int64_t T,
                             int64_t in, int64_t out, float* y, float* sumsq, void* workspace, size_t workspace_bytes,
                             void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (x_shared)
    return lowrank_shared_run(x, x_shared, w, noise, noise_stride, a_off, b_off, sign, m, T, in, out, y, sumsq,
                              workspace, workspace_bytes, stream, true);
  NOISE_REQUIRE(x && w && noise && sign, "NULL pointer argument");
  NOISE_REQUIRE(m > 0 && T > 0 && T % LTile::WTM == 0, "T = %lld must be a positive multiple of %d", (long long)T,
                LTile::WTM);
  NOISE_REQUIRE(in > 0 && in % LTile::BK == 0 && out > 0 && out % LTile::BN == 0, "in %% 32 and out %% 256 must be 0");
  NOISE_REQUIRE(a_off >= 0 && b_off >= 0 && noise_stride >= a_off + out && noise_stride >= b_off + in,
                "a / b slices outside the noise row");
  const int64_t M = m * T;
  NOISE_REQUIRE(M <= (int64_t)INT32_MAX / 4, "m * T too large");
  NOISE_REQUIRE(workspace && workspace_bytes >= noise_lowrank_workspace(m, T, in, out, 0), "workspace too small");
  float* u = (float*)workspace;
  float* part = (float*)((char*)workspace + al256((size_t)M * 4));
  hipLaunchKernelGGL(lowrank_dot_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream, (const bf16_t*)x,
                     (int)in, (int)T, noise, noise_stride, b_off, u, M);
  NOISE_LAUNCH_CHECK();
  EpiLowrank epi{(int)T, noise, noise_stride, a_off, sign, u, y, out, sumsq ? part : nullptr, (int)(out / LTile::BN)};
  NOISE_CHECK_HIP((prepare_gemm<LTile, EpiLowrank>()));
  {
    NoiseTimer tm(kTimeLowrank, stream);
    NOISE_CHECK_HIP((launch_gemm<LTile>((const bf16_t*)x, in, (const bf16_t*)w, in, (int)M, (int)out, (int)in, epi,
                                        stream)));
  }
  if (sumsq) {
    hipLaunchKernelGGL(member_part_sum_kernel, dim3((unsigned)m), dim3(256), 0, stream, part,
                       (int)(T * (out / LTile::BN)), sumsq);
    NOISE_LAUNCH_CHECK();
  }
  return NOISE_OK;
}

// ---- the plain bf16 linear ----------------------------------------------------------------------------------------

namespace noise {
// y = bf16(x W^T) (the autocast rounding of the matmul output), stored as bf16; rows past M are not stored.
struct EpiLinear {
  bf16_t* y;
  int64_t ldy;
  int M;
  static constexpr int kRows = kEpiRows;
  struct Wave {};
  struct Pre {};
  __device__ __forceinline__ void begin(int, int, int, int, Wave&) const {}
  __device__ __forceinline__ void load(int, int, int, const Wave&, Pre&) const {}
  template <int R>
  __device__ __forceinline__ void rows(int row0, int n0, int, int lane, const Wave&, const Pre&, f32x4 (&v)[R]) const {
#pragma unroll
    for (int q = 0; q < R; ++q)
      if (row0 + q < M)  // the staged values are already bf16: packing them is exact
        __builtin_nontemporal_store((u32x2{pack_bf16x2(v[q][0], v[q][1]), pack_bf16x2(v[q][2], v[q][3])}),
                                    (u32x2*)(y + (int64_t)(row0 + q) * ldy + n0 + 4 * lane));
  }
};
using LinTile = GemmShape<128, 256, 32, 2, 2, 3, 2>;  // two workgroups per CU
}  // namespace noise

extern "C" int noise_linear(const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t M, int64_t in, int64_t out,
                            uint16_t* y, int64_t ldy, void* stream) {
  NOISE_REQUIRE(x && w && y, "NULL pointer argument");
  NOISE_REQUIRE(M > 0 && M <= (int64_t)INT32_MAX / 4, "M = %lld outside [1, 2^29)", (long long)M);
  NOISE_REQUIRE(in > 0 && in % 32 == 0 && in <= 65536 && out > 0 && out % 256 == 0 && out <= 65536,
                "in = %lld must be a multiple of 32 and out = %lld a multiple of 256", (long long)in, (long long)out);
  NOISE_REQUIRE(ldx >= in && ldx % 8 == 0 && ldy >= out && ldy % 4 == 0,
                "row strides: ldx >= in, a multiple of 8; ldy >= out, a multiple of 4");
  NOISE_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)y & 7) == 0,
                "x and w must be 16-byte aligned, y 8-byte aligned");
  NOISE_REQUIRE((M + LinTile::BM - 1) / LinTile::BM <= 65535, "M too large for one launch");
  NOISE_CHECK_HIP((prepare_gemm<LinTile, EpiLinear>()));
  EpiLinear epi{(bf16_t*)y, ldy, (int)M};
  NoiseTimer tm(kTimeLinear, (hipStream_t)stream);
  NOISE_CHECK_HIP((launch_gemm<LinTile>((const bf16_t*)x, ldx, (const bf16_t*)w, in, (int)M, (int)out, (int)in, epi,
                                         (hipStream_t)stream)));
  return NOISE_OK;
}

// ---- the no-allocation variant of the shared-x path -------------------------------------------------------------

// The workspace of noise_lowrank_static: a file-scope device array, one copy per GPU (held until the process ends).
// Its name is a host-side stand-in in host code, never a device address: kernels get the address that
// hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[NOISE_LOWRANK_STATIC_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device, looked up once

// The current device's copy of `scratch`, looked up on the first call on that device (with it current).
int scratch_address(void** out) {
  int dev = -1;
  NOISE_CHECK_HIP(hipGetDevice(&dev));
  NOISE_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    NOISE_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    NOISE_REQUIRE(p != nullptr, "hipGetSymbolAddress returned NULL for the scratch array");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return NOISE_OK;
}
}  // namespace

extern "C" int noise_lowrank_static(const uint16_t* x, int32_t x_shared, const uint16_t* w, const float* noise,
                                    int64_t noise_stride, int64_t a_off, int64_t b_off, const float* sign, int64_t m,
                                    int64_t T, int64_t in, int64_t out, float* y, float* sumsq, void* stream) {
  NOISE_REQUIRE(x_shared == 1 || x_shared == 2, "noise_lowrank_static takes x_shared 1 or 2 (x [T, in] shared)");
  NOISE_REQUIRE(m > 0 && T > 0 && in > 0 && out > 0, "sizes must be positive");
  const size_t need = noise_lowrank_workspace(m, T, in, out, 1);
  NOISE_REQUIRE(need <= (size_t)NOISE_LOWRANK_STATIC_BYTES,
                "noise_lowrank_static: these sizes need %zu bytes of scratch, more than its %u-byte static array "
                "(use noise_lowrank with a workspace)", need, (unsigned)NOISE_LOWRANK_STATIC_BYTES);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != NOISE_OK) return rc;
  return lowrank_shared_run(x, x_shared, w, noise, noise_stride, a_off, b_off, sign, m, T, in, out, y, sumsq, ws,
                            (size_t)NOISE_LOWRANK_STATIC_BYTES, (hipStream_t)stream, false);
}
