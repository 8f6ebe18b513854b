// bf16 MFMA GEMM for gfx950: C[M, N] = A[M, K] . B[N, K]^T with fp32 accumulation (both operands K-contiguous:
// the x @ weight.t() of nn.Linear weights stored [out, in]). The accumulator tile goes to an epilogue functor, which
// is where the population-specific work (rank-1 member corrections, residual adds, relu^2, soft-capped CE) happens.
//
// Tiling: a workgroup computes 256 x 256 with 2 x 2 waves of 128 x 128 (4 x 4 MFMA tiles of
// v_mfma_f32_32x32x16_bf16), or one of the tiles with waves of 64 x 128: 128 x 512 with 2 x 4 waves and 64 x 512
// with 1 x 4 waves (whole 512-wide rows, for epilogues that normalize rows), 128 x 256 with 2 x 2 waves. The
// 128 x 256 and 64 x 512 tiles are sized for two workgroups per CU, so that one workgroup's epilogue runs beside
// the other's MFMAs. K advances in steps of 32 or 64 (BK) through kStages LDS stages filled by direct-to-LDS buffer
// loads (buffer_load_dwordx4 ... lds): the loads of step kt + kStages are issued as soon as every wave is done with
// step kt, so kStages - 1 steps of loads are in flight behind the MFMAs and no register holds staged data.
// One barrier per step, placed before the step's last 16-deep k-substep: the last k-substep's fragments are read
// before it and the next step's first fragments after it, so LDS latency hides behind MFMAs. 64-deep steps in two
// stages halve the barriers and waits per K against 32-deep steps in four (the same LDS): on random bf16 operands at
// M = 2^20 the 128 x 512 tile (N = 512, K = 2048) went from 929 to 1041 TFLOP/s and the 8-wave 256 x 256 tile from
// 828 to 867 (N = 2048, K = 512), with bit-identical outputs.
// An LDS row is BK bf16 = 4 or 8 16-byte chunks, swizzled by row (lds_swizzle) so that the 16 lanes of a
// ds_read_b128 phase (16 consecutive rows, one chunk) touch 16 distinct bank groups.
//
// MFMA 32x32x16 bf16 lane layout (checked on gfx950): lane l supplies A[row l%32][k 8(l/32)..8(l/32)+7] and
// B^T[col l%32][same k]; accumulator register r holds C[row (r/4)*8 + (l/32)*4 + r%4][col l%32].
// Staged epilogues take the transposed product (the weight fragment as the MFMA's A operand, the activation fragment
// as its B: both operands are "32 rows x 8 k per lane", so the fragments are the same): register r of lane l then
// holds C[row l%32][col (r/4)*8 + (l/32)*4 + r%4], four consecutive columns of one row per register quad, and the
// tile is staged with one 8-byte LDS write per quad (32 per wave of 64 x 128) instead of a 2-byte write per value
// (128). The sums are the same products in the same order: the outputs are bit-identical either way.
#pragma once

#include <type_traits>
#include <utility>

#include "common.h"

namespace noise {

constexpr int kEpiRows = 8;  // rows per epilogue group (most epilogues): consecutive and aligned, so never across a
                             // member boundary

template <int BM_, int BN_, int BK_, int WM_, int WN_, int NS_ = 4, int MINB_ = 1>
struct GemmShape {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  static constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 MFMA tiles per wave
  static constexpr int kStages = NS_;                 // LDS stages
  static constexpr int kMinBlocks = MINB_;            // workgroups per CU the registers and LDS are sized for
  static constexpr int kStageBytes = (BM + BN) * BK * 2;  // A rows then B rows
  static constexpr int kRowBytes = BK * 2;                // one LDS row: 4 (BK 32) or 8 (BK 64) 16-byte chunks
  static constexpr int kLoadRows = 1024 / kRowBytes;      // rows per 1 KB direct-to-LDS load
  static constexpr int kSub = BK / 16;                    // 16-deep k-substeps per step
  static constexpr int kADma = BM / kLoadRows / kWaves, kBDma = BN / kLoadRows / kWaves;  // loads per wave and step
  static constexpr int kDma = kADma + kBDma;
  static constexpr int kEpiLd = BN + 4;                   // bf16 staging row stride (4 elements of padding)
  static constexpr int kMainLds = kStages * kStageBytes;
  static constexpr int kEpiLds = BM * kEpiLd * 2;         // the whole tile in bf16
  static constexpr int kLdsBytes = kMainLds > kEpiLds ? kMainLds : kEpiLds;
  static constexpr int kWaveRows = BM / kWaves;           // epilogue rows per wave
  static_assert((BK == 32 || BK == 64) && WTN == 128 && (WTM == 128 || WTM == 64) && (kWaves == 4 || kWaves == 8),
                "main loop: 4 or 8 waves of 128x128 or 64x128, K steps of 32 or 64");
  static_assert(kADma * kWaves * kLoadRows == BM && kBDma * kWaves * kLoadRows == BN,
                "row groups of one load split evenly over waves");
  static_assert((BM == 256 && BN == 256) || (BM == 128 && BN == 512) || (BM == 128 && BN == 256) ||
                    (BM == 64 && BN == 512),
                "tiles: 256x256, 128x512, 128x256 or 64x512");
  static_assert(kStages >= 2 && kStages <= 4, "stages");
  static_assert((kStages - 1) * kDma < 64, "loads in flight: the vmcnt field");
  static_assert(kLdsBytes * kMinBlocks <= 160 * 1024, "LDS");
};

// One 32 x 32 x 16 product of an activation fragment a and a weight fragment b into c: C = A B^T, or with kT its
// transpose (b as the MFMA's A operand), whose accumulator holds four consecutive columns of one row per register
// quad.
template <bool kT>
__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return kT ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c, 0, 0, 0)
            : __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// The 16-byte chunk slot of LDS row r: chunk c of the row sits in slot c ^ lds_swizzle<BK>(r). With 64-byte rows
// (BK 32) a ds_read_b128 phase of 16 consecutive rows and one chunk covers rows r .. r + 15, four to a 256-byte bank
// line; (r >> 2) & 3 gives each of the four its own slot. With 128-byte rows (BK 64) two rows share a bank line, and
// (r >> 1) & 7 gives each of the 8 pairs its own slot. Either way the 16 reads hit 16 distinct groups of 4 banks.
template <int BK>
__device__ __forceinline__ int lds_swizzle(int r) {
  return BK == 32 ? (r >> 2) & 3 : (r >> 1) & 7;
}

// One 16-byte-per-lane direct-to-LDS buffer load (buffer_load_dwordx4 ... lds): lane l's 16 bytes land at
// lds + 16 l. The builtin is a gfx950 target builtin, so it is only spelled out in the device pass (the host pass
// also checks kernel template bodies and rejects it).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, unsigned char* lds, int voff, int soff) {
#if __HIP_DEVICE_COMPILE__
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)lds, 16, voff, soff, 0, 0);
#endif
}

// s_waitcnt vmcnt(n) with expcnt and lgkmcnt left alone (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8); n < 64.
template <int N>
__device__ __forceinline__ void wait_vmcnt_imm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
constexpr int kWaitLgkm0 = 0xC07F;  // s_waitcnt lgkmcnt(0)

// Workgroup barrier without a memory fence: the fence of __syncthreads would also wait for every load still in
// flight into LDS. The empty asm statements keep the compiler from moving memory accesses across it; the waits
// before it are explicit.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Hands a group of rows to the epilogue: f32x4[R] for 256-column tiles, f32x4[R][2] for 512-column tiles.
template <int H>
struct EpiRows;
template <>
struct EpiRows<1> {
  template <int R, class Epi>
  __device__ __forceinline__ static void run(const Epi& epi, int row0, int n0, int n_tile, int lane,
                                             const typename Epi::Wave& w, const typename Epi::Pre& p,
                                             f32x4 (&v)[R][1]) {
    f32x4 v1[R];
#pragma unroll
    for (int k = 0; k < R; ++k) v1[k] = v[k][0];
    epi.template rows<R>(row0, n0, n_tile, lane, w, p, v1);
  }
};
template <>
struct EpiRows<2> {
  template <int R, class Epi>
  __device__ __forceinline__ static void run(const Epi& epi, int row0, int n0, int n_tile, int lane,
                                             const typename Epi::Wave& w, const typename Epi::Pre& p,
                                             f32x4 (&v)[R][2]) {
    epi.template rows<R>(row0, n0, n_tile, lane, w, p, v);
  }
};

// One group of kEpiRows staged bf16 rows (row stride ld) to the epilogue: lane l takes columns 4l .. 4l+3 of each
// 256-column half.
template <int ld, int H, class Epi>
__device__ __forceinline__ void epi_group(const Epi& epi, const bf16_t* st, int row0, int n0, int n_tile, int lane,
                                          const typename Epi::Wave& w, const typename Epi::Pre& p) {
  constexpr int R = Epi::kRows;
  f32x4 v[R][H];
#pragma unroll
  for (int k = 0; k < R; ++k)
#pragma unroll
    for (int hh = 0; hh < H; ++hh) {
      const u32x2 q = *(const u32x2*)(st + k * ld + hh * 256 + 4 * lane);
      v[k][hh] = f32x4{__uint_as_float(q[0] << 16), __uint_as_float(q[0] & 0xFFFF0000u), __uint_as_float(q[1] << 16),
                       __uint_as_float(q[1] & 0xFFFF0000u)};
    }
  EpiRows<H>::template run<R>(epi, row0, n0, n_tile, lane, w, p, v);
}

// Instruction interleaving of the main loop's two halves (sched_group_barrier masks: 0x008 MFMA, 0x020 VMEM read,
// 0x100 LDS read; the counts must be literal constants). First half: the next k-substep's fragment reads, one after
// each MFMA. Second half: the step's direct-to-LDS loads after the first MFMAs, then the next step's fragment reads.
template <class S>
__device__ __forceinline__ void first_half_schedule() {
  if constexpr (S::TM == 4) {  // 16 MFMAs, 8 reads
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
  } else {  // 8 MFMAs, 6 reads
#pragma unroll
    for (int g = 0; g < 6; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  }
}
template <class S>
__device__ __forceinline__ void second_half_schedule() {
  if constexpr (S::TM == 4) {  // 16 MFMAs, 8 or 10 loads, 8 reads
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x020, S::kDma > 8 ? 2 : 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x020, S::kDma > 9 ? 2 : 1, 0);
#pragma unroll
    for (int g = 0; g < 6; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  } else if constexpr (S::BK == 64) {  // 8 MFMAs, 8 or 10 loads, 6 reads
    constexpr int kPairs = S::kDma - 6;  // MFMAs followed by two loads; the rest take one
    static_assert(kPairs >= 0 && kPairs <= 6, "64-deep steps: 6 to 12 loads");
#pragma unroll
    for (int g = 0; g < kPairs; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int g = kPairs; g < 6; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  } else if constexpr (S::kDma == 5) {  // 8 MFMAs, 5 loads, 6 reads
#pragma unroll
    for (int g = 0; g < 5; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  } else {  // 8 MFMAs, 6 or 9 loads, 6 reads
    constexpr int kFirst = S::kDma > 6 ? 2 : 1;  // loads after each of the first three MFMAs
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, kFirst, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  }
}

// Tile order, chosen by the epilogue. Default: each XCD's run of tiles goes in groups of 8 row panels with the column
// tiles outermost. An epilogue with `static constexpr int kNSplit = S` (S dividing the column tiles) splits the
// columns into S parts instead: the runs of the first 8 / S XCDs cover every row panel for the first part of the
// columns, and so on, each row panel's tiles of the part back to back. B's part then stays in each XCD's L2 while
// the A rows stream past, and each A row is fetched S times.
template <class E, class = void>
struct NSplit : std::integral_constant<int, 1> {};
template <class E>
struct NSplit<E, std::void_t<decltype(E::kNSplit)>> : std::integral_constant<int, E::kNSplit> {};

// An epilogue functor with `static constexpr bool kAccEpilogue = true` takes the fp32 accumulators in registers, in
// the MFMA layout, instead of the bf16 tile staged through LDS:
//   acc_epilogue<S>(acc, smem, m0, n0, m_tile, n_tile, wave, wm, wn, lane)
// with the whole LDS allocation free for its own use (every wave is past the main loop's last stage).
template <class E, class = void>
struct AccEpilogue : std::false_type {};
template <class E>
struct AccEpilogue<E, std::void_t<decltype(E::kAccEpilogue)>> : std::bool_constant<E::kAccEpilogue> {};

// A staged epilogue may define ready(Wave&): the arithmetic on begin()'s per-row loads, run once the accumulators are
// staged. An instruction that uses a loaded value makes the wave wait for the load; in begin() that wait would come
// before the staging, here the staging has covered the load's latency.
template <class E, class = void>
struct HasReady : std::false_type {};
template <class E>
struct HasReady<E, std::void_t<decltype(std::declval<const E&>().ready(std::declval<typename E::Wave&>()))>>
    : std::true_type {};

// Epilogue through LDS (every functor without an accumulator epilogue).
template <class S, class Epi>
__device__ __forceinline__ void staged_epilogue(const Epi& epi, f32x16 (&acc)[S::TM][S::TN], unsigned char* smem_raw,
                                                int M, int m0, int n0, int n_tile, int wave, int wm, int wn,
                                                int lane) {
  // The accumulators (transposed: four consecutive columns of one row per register quad) are rounded to bf16 -- the
  // rounding of the reference's bf16 autocast matmul output, to which it then adds its fp32 rank-1 term -- and staged
  // as the whole tile, 8 bytes per write; the row pitch BN + 4 puts the 32 rows of one write on distinct pairs of the
  // 64 banks (the pitch is 2 mod 64 words). Each wave then takes
  // kWaveRows rows (one member's: M and the member length are multiples of 64) in groups of Epi::kRows (8, or 4 for
  // epilogues that prefetch much per row); lane l holds
  // columns 4l .. 4l+3 of each 256-column half. The epilogue functor provides
  //   begin(row_base, n0, lane, nrows, Wave&)    loads made once per wave (noise vectors, per-row scalars by lane for
  //                                              the wave's nrows rows),
  //   ready(Wave&) (optional)                    arithmetic on those loads, after the staging,
  //   load(row0, n0, lane, const Wave&, Pre&)     the per-row data of one group (issued a group ahead),
  //   rows<R>(row0, n0, n_tile, lane, const Wave&, const Pre&, v)  the group's arithmetic and stores, with
  //   v = f32x4[R] (256-column tiles) or f32x4[R][2] (512-column tiles: columns 4l.. and 256 + 4l..).
  // The wave's per-row loads and its first group's loads are issued before the accumulators are staged, so their
  // memory latency runs behind the staging.
  bf16_t* st = (bf16_t*)smem_raw;
  constexpr int R = Epi::kRows, G = S::kWaveRows / Epi::kRows, H = S::BN / 256;
  static_assert(G % 2 == 0, "groups are processed in pairs");
  const int row_base = m0 + wave * S::kWaveRows;
  typename Epi::Wave w;
  typename Epi::Pre p0, p1;
  if (row_base < M) {
    epi.begin(row_base, n0, lane, min(S::kWaveRows, M - row_base), w);  // per-row loads by lane: lanes < nrows
    epi.load(row_base, n0, lane, w, p0);
  }
#pragma unroll
  for (int i = 0; i < S::TM; ++i)
#pragma unroll
    for (int j = 0; j < S::TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lr = wm * S::WTM + i * 32 + (lane & 31);
        const int lc = wn * S::WTN + j * 32 + q * 8 + (lane >> 5) * 4;
        *(u32x2*)(st + lr * S::kEpiLd + lc) = u32x2{pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                                                    pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
      }
  __syncthreads();
  if (row_base >= M) return;
  if constexpr (HasReady<Epi>::value) epi.ready(w);
  const bf16_t* st_wave = st + wave * S::kWaveRows * S::kEpiLd;
#pragma unroll 1
  for (int g = 0; g < G; g += 2) {
    const int r0 = row_base + g * R;
    epi.load(r0 + R, n0, lane, w, p1);
    epi_group<S::kEpiLd, H>(epi, st_wave + g * R * S::kEpiLd, r0, n0, n_tile, lane, w, p0);
    if (g + 2 < G) epi.load(r0 + 2 * R, n0, lane, w, p0);
    epi_group<S::kEpiLd, H>(epi, st_wave + (g + 1) * R * S::kEpiLd, r0 + R, n0, n_tile, lane, w, p1);
  }
}

template <class S, class Epi>
__global__ __launch_bounds__(S::kThreads, S::kMinBlocks) void gemm_nt_kernel(const bf16_t* __restrict__ A, int64_t lda,
                                                              const bf16_t* __restrict__ B, int64_t ldb, int M, int N,
                                                              int K, Epi epi) {
  constexpr int NS = S::kStages;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int kAStage = S::BM * S::BK * 2;  // A rows, then B rows
  constexpr int kStage = S::kStageBytes;

  // Workgroups are dispatched round-robin over the 8 XCDs; tiles are renumbered so that each XCD walks a contiguous
  // run of tiles (its A panels and B tiles are then fetched into one XCD's L2). Within a run, tiles go in groups of
  // up to 8 row panels with the column tiles outermost, so a B tile is reused by 8 row panels while they are
  // resident; or, with kNSplit, by column part (NSplit above).
  const int nt = gridDim.x, mt = gridDim.y, total = nt * mt;
  const int bid = blockIdx.y * nt + blockIdx.x;
  const int tile = (total % 8 == 0) ? (bid % 8) * (total / 8) + bid / 8 : bid;
  constexpr int kGroup = 8;
  constexpr int kSplit = NSplit<Epi>::value;
  int m_tile, n_tile;
  if (kSplit > 1 && nt % kSplit == 0) {
    const int ntp = nt / kSplit, per = mt * ntp;
    const int part = tile / per, r = tile % per;
    m_tile = r / ntp;
    n_tile = part * ntp + r % ntp;
  } else {
    const int grp = tile / (kGroup * nt), in_grp = tile % (kGroup * nt);
    const int grp_rows = min(kGroup, mt - grp * kGroup);
    m_tile = grp * kGroup + in_grp % grp_rows;
    n_tile = in_grp / grp_rows;
  }
  const int m0 = m_tile * S::BM, n0 = n_tile * S::BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, so in a scalar register
  const int wm = wave / S::WN, wn = wave % S::WN;
  const int a_rows = min(S::BM, M - m0), b_rows = min(S::BN, N - n0);

  // Buffer resources over this tile's rows. The row goes in the per-lane offset, which the range check covers, so
  // rows past the last one read as zeros; the K step goes in the scalar offset.
  const __amdgpu_buffer_rsrc_t a_rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)(A + (int64_t)m0 * lda), 0, a_rows * (int)lda * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t b_rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)(B + (int64_t)n0 * ldb), 0, b_rows * (int)ldb * 2, 0x00020000);

  // One direct-to-LDS load fills 1 KB = kLoadRows rows of kRowBytes: lane l writes LDS bytes 16 l .. 16 l + 15,
  // i.e. row l / (chunks per row), slot l % (chunks per row), so it fetches the global chunk that the row's swizzle
  // puts in that slot. Wave w fills row groups w kADma .. (w + 1) kADma - 1 of A and w kBDma .. (w + 1) kBDma - 1
  // of B.
  constexpr int kChunks = S::kRowBytes / 16;
  const int drow = lane / kChunks, dslot = lane % kChunks;
  auto load_off = [&](int g, int ld) {
    const int r = g * S::kLoadRows + drow;
    return (r * ld + (dslot ^ lds_swizzle<S::BK>(r)) * 8) * 2;
  };
  int a_vo[S::kADma], b_vo[S::kBDma];
#pragma unroll
  for (int j = 0; j < S::kADma; ++j) a_vo[j] = load_off(wave * S::kADma + j, (int)lda);
#pragma unroll
  for (int j = 0; j < S::kBDma; ++j) b_vo[j] = load_off(wave * S::kBDma + j, (int)ldb);
  const int nk = K / S::BK;
  // Steps past the last one are issued too, with an offset past the buffer's end: the hardware returns zeros
  // without a memory access, and every step has the same number of loads in flight.
  auto dma = [&](int kt, int stage) {
    const int koff = kt * S::BK * 2;
    const int oob = kt < nk ? 0 : (1 << 30);
    unsigned char* a_base = smem_raw + stage * kStage + wave * S::kADma * 1024;
    unsigned char* b_base = smem_raw + stage * kStage + kAStage + wave * S::kBDma * 1024;
#pragma unroll
    for (int j = 0; j < S::kADma; ++j)
      dma16(a_rsrc, a_base + j * 1024, a_vo[j] + oob, koff);
#pragma unroll
    for (int j = 0; j < S::kBDma; ++j)
      dma16(b_rsrc, b_base + j * 1024, b_vo[j] + oob, koff);
  };

  // Fragment offsets of k-substep kk: row (lane & 31) of a 32-row tile, chunk 2 kk + (lane >> 5), in its swizzled
  // slot (the swizzle repeats every 16 rows, so it holds for every 32-row tile of the stage).
  const int xs = lds_swizzle<S::BK>(lane & 31);
  int fa_off[S::kSub], fb_off[S::kSub];
#pragma unroll
  for (int kk = 0; kk < S::kSub; ++kk) {
    const int ch = ((2 * kk + (lane >> 5)) ^ xs) * 16;
    fa_off[kk] = (wm * S::WTM + (lane & 31)) * S::kRowBytes + ch;
    fb_off[kk] = kAStage + (wn * S::WTN + (lane & 31)) * S::kRowBytes + ch;
  }
  auto frag = [&](int off) { return *(const bf16x8*)(smem_raw + off); };
  constexpr int kTileStride = 32 * S::kRowBytes;  // bytes between the 32-row MFMA tiles of a stage

  f32x16 acc[S::TM][S::TN];  // first written by step 0's first MFMAs, which take a zero accumulator
  constexpr bool kTr = !AccEpilogue<Epi>::value;  // staged epilogues take the transposed tile

  // Prologue: steps 0 .. NS - 1 in flight; stage 0 visible; its first k-substep's fragments read.
#pragma unroll
  for (int s = 0; s < NS; ++s) dma(s, s);
  wait_vmcnt_imm<(NS - 1) * S::kDma>();
  lds_barrier();
  bf16x8 fa[2][S::TM], fb[2][S::TN];  // fragments of alternate k-substeps
#pragma unroll
  for (int i = 0; i < S::TM; ++i) fa[0][i] = frag(fa_off[0] + i * kTileStride);
#pragma unroll
  for (int j = 0; j < S::TN; ++j) fb[0][j] = frag(fb_off[0] + j * kTileStride);

  // Step kt on stage kt % NS: for each k-substep but the last, read the next k-substep and multiply this one; wait
  // for this wave's reads and for stage kt + 1's loads, barrier (everyone is then past its reads of stage kt, and
  // stage kt + 1 is visible); refill stage kt % NS with step kt + NS; read the next step's k-substep 0 and multiply
  // the last k-substep.
  // The reads and loads of each part are spread between its MFMAs (one per MFMA), so that neither the LDS nor the
  // texture-address queue sees a burst.
  // Step 0 is peeled: its first MFMAs take the inline constant 0 as the accumulator, so the accumulators need no
  // zeroing moves.
  auto step = [&](int kt, auto first) {
    const int pb = (kt % NS) * kStage;
#pragma unroll
    for (int kk = 0; kk + 1 < S::kSub; ++kk) {
      const int nx = (kk + 1) & 1, cu = kk & 1;
#pragma unroll
      for (int i = 0; i < S::TM; ++i) fa[nx][i] = frag(fa_off[kk + 1] + pb + i * kTileStride);
#pragma unroll
      for (int j = 0; j < S::TN; ++j) fb[nx][j] = frag(fb_off[kk + 1] + pb + j * kTileStride);
#pragma unroll
      for (int i = 0; i < S::TM; ++i)
#pragma unroll
        for (int j = 0; j < S::TN; ++j)
          acc[i][j] = mma<kTr>(fa[cu][i], fb[cu][j], decltype(first)::value && kk == 0 ? f32x16{} : acc[i][j]);
      first_half_schedule<S>();
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    wait_vmcnt_imm<(NS - 2) * S::kDma>();  // stage kt + 1 has landed (the loads of kt + 2, kt + 3 may still fly)
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    dma(kt + NS, kt % NS);
    const int nb = ((kt + 1) % NS) * kStage;
    constexpr int kLast = (S::kSub - 1) & 1;  // the last k-substep's fragment set; the next step's first goes in 0
#pragma unroll
    for (int i = 0; i < S::TM; ++i) fa[0][i] = frag(fa_off[0] + nb + i * kTileStride);
#pragma unroll
    for (int j = 0; j < S::TN; ++j) fb[0][j] = frag(fb_off[0] + nb + j * kTileStride);
#pragma unroll
    for (int i = 0; i < S::TM; ++i)
#pragma unroll
      for (int j = 0; j < S::TN; ++j)
        acc[i][j] = mma<kTr>(fa[kLast][i], fb[kLast][j], acc[i][j]);
    second_half_schedule<S>();
    __builtin_amdgcn_sched_barrier(0);
  };
  step(0, std::true_type{});
  for (int kt = 1; kt < nk; ++kt) step(kt, std::false_type{});
  wait_vmcnt_imm<0>();  // the loads issued past the last step have landed
  __syncthreads();      // every wave is done with the stages before the epilogue reuses the LDS

  if constexpr (AccEpilogue<Epi>::value)
    epi.template acc_epilogue<S>(acc, smem_raw, m0, n0, m_tile, n_tile, wave, wm, wn, lane);
  else
    staged_epilogue<S>(epi, acc, smem_raw, M, m0, n0, n_tile, wave, wm, wn, lane);
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
