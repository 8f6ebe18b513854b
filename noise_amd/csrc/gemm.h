// bf16 MFMA GEMM for gfx950: C[M, N] = A[M, K] . B[N, K]^T with fp32 accumulation (both operands K-contiguous:
// the x @ weight.t() of nn.Linear weights stored [out, in]). The accumulator tile goes to an epilogue functor, which
// is where the population-specific work (rank-1 member corrections, residual adds, relu^2, soft-capped CE) happens.
//
// Tiling: a workgroup computes BM x BN with WM x WN waves; a wave owns (BM/WM) x (BN/WN) as 32x32 MFMA tiles
// (v_mfma_f32_32x32x16_bf16). K advances in BK steps through two LDS buffers: the next tile's global loads are
// issued before the current tile's MFMAs, and stored to the other buffer after them (one barrier per step).
// LDS rows are BK bf16 = BK/8 16-byte chunks; chunk c of row r is stored at c ^ (r & 7), so the 8 rows a
// ds_read_b128 phase touches fall on distinct banks.
//
// MFMA 32x32x16 bf16 lane layout (checked on gfx950): lane l supplies A[row l%32][k 8(l/32)..8(l/32)+7] and
// B^T[col l%32][same k]; accumulator register r holds C[row (r/4)*8 + (l/32)*4 + r%4][col l%32].
#pragma once

#include "common.h"

namespace noise {

constexpr int kEpiRows = 8;  // rows per epilogue group: consecutive, 8-aligned, so never across a member boundary

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct GemmShape {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int kThreads = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  static constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 MFMA tiles per wave
  static constexpr int kChunks = BK / 8;              // 16-byte chunks per LDS row
  static constexpr int kAVec = BM * kChunks / kThreads;  // 16-byte global loads per thread
  static constexpr int kBVec = BN * kChunks / kThreads;
  static constexpr int kEpiLd = BN + 16;                // bf16 staging row stride (16 elements of padding)
  static constexpr int kMainLds = 2 * (BM + BN) * BK * 2;
  static constexpr int kEpiLds = BM * kEpiLd * 2;         // the whole tile in bf16
  static constexpr int kLdsBytes = kMainLds > kEpiLds ? kMainLds : kEpiLds;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
  static_assert(BK % 16 == 0 && kChunks <= 8 && kChunks >= 2, "BK in {16, 32, 64}");
  static_assert((BM * kChunks) % kThreads == 0 && (BN * kChunks) % kThreads == 0, "tile loads must divide threads");
};

template <int kChunks>
__device__ __forceinline__ int swz(int row, int chunk) {
  return chunk ^ (row & (kChunks - 1));
}

// Row-major [rows x BK] bf16 tile of a K-contiguous matrix -> registers (16 bytes per vector).
template <class S, int kVec>
__device__ __forceinline__ void load_tile(const bf16_t* __restrict__ g, int64_t ld, int row0, int rows_valid, int k0,
                                          u32x4 (&r)[kVec]) {
#pragma unroll
  for (int i = 0; i < kVec; ++i) {
    const int v = threadIdx.x + i * S::kThreads;
    const int row = v / S::kChunks, chunk = v % S::kChunks;
    if (row < rows_valid)
      r[i] = *(const u32x4*)(g + (int64_t)(row0 + row) * ld + k0 + chunk * 8);
    else
      r[i] = u32x4{0u, 0u, 0u, 0u};
  }
}

template <class S, int kVec>
__device__ __forceinline__ void store_tile(bf16_t* lds, const u32x4 (&r)[kVec]) {
#pragma unroll
  for (int i = 0; i < kVec; ++i) {
    const int v = threadIdx.x + i * S::kThreads;
    const int row = v / S::kChunks, chunk = v % S::kChunks;
    *(u32x4*)(lds + row * S::BK + swz<S::kChunks>(row, chunk) * 8) = r[i];
  }
}

template <class S>
__device__ __forceinline__ bf16x8 read_frag(const bf16_t* lds, int row, int kchunk) {
  return *(const bf16x8*)(lds + row * S::BK + swz<S::kChunks>(row, kchunk) * 8);
}

template <class S, class Epi>
__global__ __launch_bounds__(S::kThreads) void gemm_nt_kernel(const bf16_t* __restrict__ A, int64_t lda,
                                                              const bf16_t* __restrict__ B, int64_t ldb, int M, int N,
                                                              int K, Epi epi) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  // stage s: A tile at lds + s * kStage, B tile at lds + s * kStage + BM * BK (offsets, not a pointer array, so the
  // accesses stay ds_read / ds_write)
  bf16_t* lds = (bf16_t*)smem_raw;
  constexpr int kStage = (S::BM + S::BN) * S::BK;

  // Workgroups are dispatched round-robin over the 8 XCDs; tiles are renumbered so that each XCD walks a contiguous
  // run of tiles (its A panels and B tiles are then fetched into one XCD's L2).
  // Within a run, tiles go in groups of up to 8 row panels with the column tiles outermost, so a B tile is reused
  // by 8 row panels while they are resident (the 4 MB lm_head weight does not fit one L2 next to its A panels).
  const int nt = gridDim.x, mt = gridDim.y, total = nt * mt;
  const int bid = blockIdx.y * nt + blockIdx.x;
  const int tile = (total % 8 == 0) ? (bid % 8) * (total / 8) + bid / 8 : bid;
  constexpr int kGroup = 8;
  const int grp = tile / (kGroup * nt), in_grp = tile % (kGroup * nt);
  const int grp_rows = min(kGroup, mt - grp * kGroup);
  const int m_tile = grp * kGroup + in_grp % grp_rows, n_tile = in_grp / grp_rows;
  const int m0 = m_tile * S::BM, n0 = n_tile * S::BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / S::WN, wn = wave % S::WN;
  const int a_rows = min(S::BM, M - m0), b_rows = min(S::BN, N - n0);

  f32x16 acc[S::TM][S::TN];
#pragma unroll
  for (int i = 0; i < S::TM; ++i)
#pragma unroll
    for (int j = 0; j < S::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  u32x4 ra[S::kAVec], rb[S::kBVec];
  load_tile<S, S::kAVec>(A, lda, m0, a_rows, 0, ra);
  load_tile<S, S::kBVec>(B, ldb, n0, b_rows, 0, rb);
  store_tile<S, S::kAVec>(lds, ra);
  store_tile<S, S::kBVec>(lds + S::BM * S::BK, rb);
  __syncthreads();

  const int nk = K / S::BK;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      load_tile<S, S::kAVec>(A, lda, m0, a_rows, (kt + 1) * S::BK, ra);
      load_tile<S, S::kBVec>(B, ldb, n0, b_rows, (kt + 1) * S::BK, rb);
    }
    const bf16_t* as = lds + cur * kStage;
    const bf16_t* bs = as + S::BM * S::BK;
    // fragments of k-substep kk + 1 are read while the MFMAs of kk run
    bf16x8 fa[2][S::TM], fb[2][S::TN];
#pragma unroll
    for (int i = 0; i < S::TM; ++i) fa[0][i] = read_frag<S>(as, wm * S::WTM + i * 32 + (lane & 31), (lane >> 5));
#pragma unroll
    for (int j = 0; j < S::TN; ++j) fb[0][j] = read_frag<S>(bs, wn * S::WTN + j * 32 + (lane & 31), (lane >> 5));
#pragma unroll
    for (int kk = 0; kk < S::BK / 16; ++kk) {
      const int c = kk & 1;
      if (kk + 1 < S::BK / 16) {
#pragma unroll
        for (int i = 0; i < S::TM; ++i)
          fa[c ^ 1][i] = read_frag<S>(as, wm * S::WTM + i * 32 + (lane & 31), (kk + 1) * 2 + (lane >> 5));
#pragma unroll
        for (int j = 0; j < S::TN; ++j)
          fb[c ^ 1][j] = read_frag<S>(bs, wn * S::WTN + j * 32 + (lane & 31), (kk + 1) * 2 + (lane >> 5));
      }
#pragma unroll
      for (int i = 0; i < S::TM; ++i)
#pragma unroll
        for (int j = 0; j < S::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[c][i], fb[c][j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) {
      store_tile<S, S::kAVec>(lds + (cur ^ 1) * kStage, ra);
      store_tile<S, S::kBVec>(lds + (cur ^ 1) * kStage + S::BM * S::BK, rb);
    }
    __syncthreads();
  }
  // Epilogue through LDS. The accumulators are rounded to bf16 -- the rounding of the reference's bf16 autocast matmul
  // output, to which it then adds its fp32 rank-1 term -- and staged as the whole 256 x 256 tile. Each wave then takes
  // 64 rows in groups of kEpiRows (lane l holds columns 4l .. 4l+3) and hands a group to the epilogue, which issues
  // all of the group's loads before it computes and stores. Rows past M are skipped.
  static_assert(S::BN == 256 && S::kThreads == 256 && S::BM == 256, "row epilogue: 256 x 256 tiles, 4 waves");
  bf16_t* st = (bf16_t*)smem_raw;
#pragma unroll
  for (int i = 0; i < S::TM; ++i)
#pragma unroll
    for (int j = 0; j < S::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = wm * S::WTM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        st[lr * S::kEpiLd + wn * S::WTN + j * 32 + (lane & 31)] = f32_to_bf16(acc[i][j][r]);
      }
  __syncthreads();
  constexpr int R = kEpiRows;
#pragma unroll 1
  for (int g = 0; g < 64 / R; ++g) {
    const int lr0 = wave * 64 + g * R;
    if (m0 + lr0 >= M) break;  // M % 8 == 0: a group is all valid or all past the end
    f32x4 v[R];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const u32x2 p = *(const u32x2*)(st + (lr0 + k) * S::kEpiLd + 4 * lane);
      v[k] = f32x4{__uint_as_float(p[0] << 16), __uint_as_float(p[0] & 0xFFFF0000u), __uint_as_float(p[1] << 16),
                   __uint_as_float(p[1] & 0xFFFF0000u)};
    }
    epi.template rows<R>(m0 + lr0, n0, n_tile, lane, v);
  }
}

// Row / column of accumulator element (i, j, r) for this lane.
__device__ __forceinline__ int acc_row(int row0, int i, int r, int lane) {
  return row0 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
}
__device__ __forceinline__ int acc_col(int col0, int j, int lane) { return col0 + j * 32 + (lane & 31); }

template <class S, class Epi>
static inline hipError_t launch_gemm(const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, int M, int N, int K,
                                     const Epi& epi, hipStream_t stream) {
  dim3 grid((N + S::BN - 1) / S::BN, (M + S::BM - 1) / S::BM);
  hipLaunchKernelGGL((gemm_nt_kernel<S, Epi>), grid, dim3(S::kThreads), S::kLdsBytes, stream, A, lda, B, ldb, M, N,
                     K, epi);
  return hipGetLastError();
}

template <class S, class Epi>
static inline hipError_t prepare_gemm() {
  return hipFuncSetAttribute((const void*)gemm_nt_kernel<S, Epi>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             S::kLdsBytes);
}

}  // namespace noise
