// bf16 MFMA GEMM for gfx950: C[M, N] = A[M, K] . B[N, K]^T with fp32 accumulation (both operands K-contiguous:
// the x @ weight.t() of nn.Linear weights stored [out, in]). The accumulator tile goes to an epilogue functor, which
// is where the population-specific work (rank-1 member corrections, residual adds, relu^2, soft-capped CE) happens.
//
// Tiling: a workgroup computes BM x BN with WM x WN waves; a wave owns (BM/WM) x (BN/WN) as 32x32 MFMA tiles
// (v_mfma_f32_32x32x16_bf16). K advances in BK steps through two LDS buffers: the next step's buffer loads are issued
// before the current step's MFMAs and stored to the other buffer after them (one barrier per step).
// LDS rows are BK bf16 = BK/8 16-byte chunks, XOR-swizzled (swz below) so that every ds_read_b128 / ds_write_b128
// phase is free of bank conflicts.
//
// MFMA 32x32x16 bf16 lane layout (checked on gfx950): lane l supplies A[row l%32][k 8(l/32)..8(l/32)+7] and
// B^T[col l%32][same k]; accumulator register r holds C[row (r/4)*8 + (l/32)*4 + r%4][col l%32].
#pragma once

#include <type_traits>

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

// 16-byte chunk c of LDS row r is stored at c ^ ((r >> 1) & (kChunks - 1)): a ds_read_b128 / ds_write_b128 phase
// (16 lanes, 256 bytes) then touches 16 distinct bank groups both for fragment reads (16 consecutive rows, one chunk)
// and for tile stores (2 rows x 8 chunks).
template <int kChunks>
__device__ __forceinline__ int swz(int row, int chunk) {
  return chunk ^ ((row >> 1) & (kChunks - 1));
}

template <class S, class Epi>
__global__ __launch_bounds__(S::kThreads) void gemm_nt_kernel(const bf16_t* __restrict__ A, int64_t lda,
                                                              const bf16_t* __restrict__ B, int64_t ldb, int M, int N,
                                                              int K, Epi epi) {
  static_assert(S::BK == 64, "main loop: 8 chunks of 16 bytes per LDS row");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  // LDS (bytes): A stage s at s * kAStage, B stage s at 2 * kAStage + s * kBStage. Every LDS access below is a
  // per-lane base register plus an immediate offset (< 64 KB).
  constexpr int kAStage = S::BM * S::BK * 2, kBStage = S::BN * S::BK * 2;

  // Workgroups are dispatched round-robin over the 8 XCDs; tiles are renumbered so that each XCD walks a contiguous
  // run of tiles (its A panels and B tiles are then fetched into one XCD's L2). Within a run, tiles go in groups of
  // up to 8 row panels with the column tiles outermost, so a B tile is reused by 8 row panels while they are
  // resident (the 4 MB lm_head weight does not fit one L2 next to its A panels).
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

  // Buffer resources over this tile's rows: reads past the last row return zeros. The K step and the row pass go
  // in the scalar offset, so a load costs no vector address arithmetic.
  const __amdgpu_buffer_rsrc_t a_rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)(A + (int64_t)m0 * lda), 0, a_rows * (int)lda * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t b_rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)(B + (int64_t)n0 * ldb), 0, b_rows * (int)ldb * 2, 0x00020000);
  constexpr int kRowsPerPass = S::kThreads / S::kChunks;  // rows covered by one 16-byte load per thread
  const int lrow = threadIdx.x / S::kChunks, lchunk = threadIdx.x % S::kChunks;
  const int a_voff = (lrow * (int)lda + lchunk * 8) * 2, b_voff = (lrow * (int)ldb + lchunk * 8) * 2;
  const int a_pass = kRowsPerPass * (int)lda * 2, b_pass = kRowsPerPass * (int)ldb * 2;
  const int st_off = (lrow * S::BK + swz<S::kChunks>(lrow, lchunk) * 8) * 2;  // rows lrow + 32 i share the swizzle

  // fragment offsets for each 16-deep k-substep (row bits 1..3 = lane bits 1..3)
  const int xs = ((lane & 31) >> 1) & 7;
  int fa_off[S::BK / 16], fb_off[S::BK / 16];
#pragma unroll
  for (int kk = 0; kk < S::BK / 16; ++kk) {
    const int ch = ((2 * kk + (lane >> 5)) ^ xs) * 16;
    fa_off[kk] = (wm * S::WTM + (lane & 31)) * S::BK * 2 + ch;
    fb_off[kk] = 2 * kAStage + (wn * S::WTN + (lane & 31)) * S::BK * 2 + ch;
  }

  f32x16 acc[S::TM][S::TN];
#pragma unroll
  for (int i = 0; i < S::TM; ++i)
#pragma unroll
    for (int j = 0; j < S::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  u32x4 ra[S::kAVec], rb[S::kBVec];
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < S::kAVec; ++i)
      ra[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_voff, i * a_pass + kt * S::BK * 2, 0));
#pragma unroll
    for (int i = 0; i < S::kBVec; ++i)
      rb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, b_voff, i * b_pass + kt * S::BK * 2, 0));
  };
  auto lstore = [&](int stage) {
    const int sa = stage * kAStage, sb = 2 * kAStage + stage * kBStage;
#pragma unroll
    for (int i = 0; i < S::kAVec; ++i) *(u32x4*)(smem_raw + sa + st_off + i * kRowsPerPass * S::BK * 2) = ra[i];
#pragma unroll
    for (int i = 0; i < S::kBVec; ++i) *(u32x4*)(smem_raw + sb + st_off + i * kRowsPerPass * S::BK * 2) = rb[i];
  };
  auto frag = [&](int off) { return *(const bf16x8*)(smem_raw + off); };

  const int nk = K / S::BK;
  gload(0);
  lstore(0);
  __syncthreads();

  // K steps on LDS stage P = kt & 1: issue the next step's loads, run the MFMAs (fragments of k-substep kk + 1 are
  // read while those of kk multiply), store the loaded step to stage P ^ 1, barrier
  for (int kt = 0; kt < nk; ++kt) {
    const int P = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) gload(kt + 1);
    const int pa = P * kAStage, pb = P * kBStage;
    bf16x8 fa[2][S::TM], fb[2][S::TN];
#pragma unroll
    for (int i = 0; i < S::TM; ++i) fa[0][i] = frag(fa_off[0] + pa + i * 32 * S::BK * 2);
#pragma unroll
    for (int j = 0; j < S::TN; ++j) fb[0][j] = frag(fb_off[0] + pb + j * 32 * S::BK * 2);
#pragma unroll
    for (int kk = 0; kk < S::BK / 16; ++kk) {
      const int c = kk & 1;
      if (kk + 1 < S::BK / 16) {
#pragma unroll
        for (int i = 0; i < S::TM; ++i) fa[c ^ 1][i] = frag(fa_off[kk + 1] + pa + i * 32 * S::BK * 2);
#pragma unroll
        for (int j = 0; j < S::TN; ++j) fb[c ^ 1][j] = frag(fb_off[kk + 1] + pb + j * 32 * S::BK * 2);
      }
#pragma unroll
      for (int i = 0; i < S::TM; ++i)
#pragma unroll
        for (int j = 0; j < S::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[c][i], fb[c][j], acc[i][j], 0, 0, 0);
    }
    if (more) lstore(P ^ 1);
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
