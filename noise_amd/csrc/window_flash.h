// Windowed causal flash kernel for head_dim 64 on gfx950, shared by three passes:
//
//   kAttn   out_o = sum_i softmax_i(x_o . y_i / 8) v_i over 0 <= o - i <= W   (attention forward; x = q, y = k)
//           utils/model.py:17-31
//   kLse    lse_o = log sum_i exp(x_o . y_i / 8) over the same window          (credit LSE pass; x = q, y = k)
//           train/speedrun/moment_kernels.py:79-110
//   kCredit out_o = sum_i exp(x_o . y_i / 8 - lse_i) v_i over 0 <= i - o <= W  (credit value pass; x = k, y = q,
//           v = the fp32 source as bf16 high (+ low) parts)  train/speedrun/moment_kernels.py:612-661
//   kCenter lse_o as kLse, and center_o = sum_i softmax_i(x_o . y_i / 8) (hub_o . v_i) over 0 <= o - i <= W
//           (credit key-context pass; x = q, y = k, v = values)  train/speedrun/moment_kernels.py:79-110
//
// A workgroup owns 128 OG outputs of one (batch, head) row: 4 waves x OG groups of 32 outputs.
// Inputs stream through two LDS stages in tiles of 64; the next tile's global loads are issued before the current
// tile's MFMAs (one barrier per tile): bf16 tiles as direct-to-LDS loads, kCredit's fp32 values through registers.
// Scores are computed transposed, S^T[i, o] = y_i . x_o (v_mfma_f32_32x32x16_bf16,
// y from LDS as the A operand, x in registers as the B operand): the accumulator layout of S^T (lane = output l%32,
// registers = 16 inputs) is exactly the B-operand layout of O^T[d, o] += V^T[d, i] P^T[i, o], so probabilities go
// from score registers to the value MFMA without an LDS round trip. Every y and V fragment read from LDS feeds all
// output groups of a wave. y is staged row-major in 16-byte chunks XOR-swizzled by row pairs, so a quarter-wave's
// row reads hit distinct banks. Values are staged row-major too, kAttn's and kCenter's like y, kCredit's fp32 source
// as bf16 high and, on request, low parts in 8-byte units swizzled for the transposing LDS read (ds_read_b64_tr_b16,
// vt_slot) that builds the V^T operand fragments.
//
// kCenter computes the value scores the same way as the logits, S2^T[i, o] = v_i . hub_o (v staged in LDS like y,
// hub in registers like x), and accumulates sum_i p_i s2_i beside sum_i p_i with fp32 probabilities.
//
// kAttn with OPT, bounded: the model normalizes q and k (RMS over 64 channels, so |q| = |k| <= 8 and
// |q . k / 8| <= 8); softmax weights are then exp(s) in [e^-8, e^8] (fp32 and bf16 hold them exactly enough) with
// no running maximum and no rescaling. The scale log2(e) / 8 is folded into q's fragments, so a weight is one exp2 of
// the score MFMA's output.
#pragma once

#include <type_traits>

#include "common.h"
#include "rng.h"

namespace noise {

enum FlashMode { kAttn = 0, kLse = 1, kCredit = 2, kCenter = 3 };

struct FlashArgs {
  const bf16_t* x;  // output-side vectors [batch, T, heads, 64] with strides below
  const bf16_t* y;  // input-side vectors
  const void* v;    // values: bf16 (kAttn, kCenter) or fp32 (kCredit)
  const bf16_t* hub;  // kCenter: per-output vectors, same strides as x
  float* center_out;  // kCenter: [batch * heads, T]
  int64_t x_sb, x_st, y_sb, y_st, v_sb, v_st;  // strides (elements) of batch and token; head h at +64 h
  const float* lse_in;  // kCredit: [batch * heads, T]
  void* out;            // kAttn: bf16 [batch, T, heads*64] (strides o_sb, o_st); kCredit: fp32 likewise
  int64_t o_sb, o_st;
  float* lse_out;       // kAttn / kLse: [batch * heads, T] (optional for kAttn)
  float* xb_out;        // kAttn (optional): [batch, T, heads] = out_o . xb_vec[h*64 ..] (rank-1 partial dots)
  const float* xb_vec;  // kAttn: per-batch vector base, batch b uses xb_vec + xb_row[b] * xb_stride
  const int32_t* xb_row;  // entries outside [0, xb_rows) read row 0 (the forward marks such a member's loss NaN)
  int64_t xb_stride, xb_rows;
  int32_t heads, T, window;
  // kAttn: the direct draws' jitter of the output (jit_sigma 0: none). Batch entry b is draw jit_draw0 + b / jit_n_seq
  // of token row jit_seq[b]; the jitter of output o, channel c of the heads * 64 comes from rng.h dust_noise_quad.
  float jit_sigma;
  uint32_t jit_site;
  uint64_t jit_seed;
  int32_t jit_draw0, jit_n_seq;
  const int32_t* jit_seq;
  // kCredit (launched with heads = 1, so row b is one (batch, head) row of q, k and lse): the value source's and the
  // output's rows may sit by token instead, row b at head b % v_div of token row b / v_div (stride v_sb), and at head
  // b % o_div of output row o_map[b / o_div] (or b / o_div without a map; stride o_sb). 0 or 1: row b itself.
  int32_t v_div, o_div;
  const int32_t* o_map;
  // kAttn: an operand shared by groups of batch entries: with a period p > 0, batch entry b reads entry b % p of x, y
  // or v (0: its own), so per-draw batches [draws * p] can read one clean copy of the operands they do not jitter
  int32_t x_period, y_period, v_period;
};

constexpr int kFlashBI = 64;
constexpr int kWaitVm0 = 0x0F70;  // s_waitcnt vmcnt(0), expcnt and lgkmcnt left alone (gfx9 encoding)

// One 16-byte direct-to-LDS load per lane (buffer_load_dwordx4 ... lds): lane l of the wave fills LDS bytes
// lds + 16 l .. lds + 16 l + 15 (lds wave-uniform). The LDS address goes in as a plain integer: given the array it
// points into, the compiler makes the next LDS reads of that array wait for the load (it does not tell the two
// stages apart), which would put the next tile's load latency inside every iteration. The loop orders the stages
// itself (vmcnt(0) and a barrier at the end of each tile).
__device__ __forceinline__ void flash_dma16(__amdgpu_buffer_rsrc_t rsrc, void* lds, int voff, int soff) {
#if __HIP_DEVICE_COMPILE__
  uint32_t addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  asm volatile("" : "+s"(addr));
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(uintptr_t)addr, 16, voff,
                                           soff, 0, 0);
#endif
}

// LDS element index of 8-byte unit u (channels 4u .. 4u+3) of value row r in the layout read by ds_read_b64_tr_b16.
// One such read has each half-wave take 8 units of 4 consecutive rows; slot u ^ 4 (r & 3) puts those 32 pieces on
// 64 distinct banks (64 banks of 4 bytes; rows of 128 bytes alternate between the two bank halves). A 16-byte chunk
// (units 2c, 2c+1) stays contiguous, so row stores by 8 or 16 bytes are conflict-free as well.
__device__ __forceinline__ int vt_slot(int r, int u) { return r * 64 + ((u ^ ((r & 3) << 2)) << 2); }
template <int OG> struct FlashTile { static constexpr int BO = 4 * 32 * OG; };  // outputs per workgroup
constexpr float kLog2e = 1.4426950408889634f;


// The part of a tile staged through registers: kCredit's fp32 values (4 16-byte chunks, 4 channels each, per
// thread) and LSE values; the other modes load straight to LDS.
template <int MODE>
struct FlashStage {};
template <>
struct FlashStage<kCredit> {
  f32x4 v[4];
  float lse;
};

// Waves per SIMD the registers are sized for. Bounded attention (the model's forward) fits 128 VGPRs, so four
// workgroups share a CU (4 x 32 KB of LDS); the credit value pass fits 168 (three workgroups, 3 x 48.5 KB); the other
// modes need more registers and keep two.
template <int MODE, bool OPT>
constexpr int kFlashOccupancy = (MODE == kAttn && OPT) ? 4 : (MODE == kCredit && !OPT ? 3 : 2);

// OPT: kAttn's and kLse's bounded softmax; kCredit's value source as bf16 high and low parts (otherwise the high part
// only).
template <int MODE, bool OPT, int OG>
__global__ __launch_bounds__(256, (kFlashOccupancy<MODE, OPT>)) void window_flash_kernel(FlashArgs a) {
  constexpr int kBO = FlashTile<OG>::BO;
  __shared__ __align__(16) bf16_t ys[2][64 * 64];
  __shared__ __align__(16) bf16_t vt_hi[2][64 * 64];
  __shared__ __align__(16) bf16_t vt_lo[MODE == kCredit && OPT ? 2 : 1][MODE == kCredit && OPT ? 64 * 64 : 4];
  __shared__ float lse_s[2][64];

  const int T = a.T, W = a.window;
  const int n_tiles = (T + kBO - 1) / kBO;
  // Workgroup order. When every row's inputs together fit well inside the 256 MB Infinity Cache, the tiles are
  // dispatched heaviest first across all rows (tile rank outer, rows inner): a launch of a few rounds of workgroups
  // then ends on its lightest tiles instead of on a late heavy one. Otherwise workgroups go round-robin to the 8 XCDs
  // and, when the (batch, head) rows divide by 8, XCD x takes rows x, x + 8, ... and runs every output tile of a row
  // back to back, so the row's inputs (512 KB at T = 2048) stay in its L2.
  const int64_t n_rows = (int64_t)gridDim.y * gridDim.z;
  const int64_t bid = blockIdx.x + (int64_t)n_tiles * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
  constexpr int64_t kInBytes = 128 + (MODE == kCredit ? 256 : MODE == kLse ? 0 : 128);  // input bytes per token
  int64_t row_idx;
  int tile_idx;
  if (n_rows * T * kInBytes <= (128ll << 20)) {
    tile_idx = (int)(bid / n_rows);
    row_idx = bid % n_rows;
  } else if (n_rows % 8 == 0) {
    const int64_t slot = bid >> 3;
    row_idx = (bid & 7) + 8 * (slot / n_tiles);
    tile_idx = (int)(slot % n_tiles);
  } else {
    row_idx = bid / n_tiles;
    tile_idx = (int)(bid % n_tiles);
  }
  // heaviest output tiles first (kAttn / kLse: late outputs see the most inputs; kCredit: early ones)
  const int tile = (MODE == kCredit) ? tile_idx : n_tiles - 1 - tile_idx;
  const int head = (int)(row_idx % gridDim.y);
  const int64_t b = row_idx / gridDim.y;
  const int o0 = tile * kBO;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, col = lane & 31;
  const int ow = o0 + wave * 32 * OG;  // this wave's first output
  const bool wave_live = ow < T;       // T % 128 == 0, so a live wave's outputs are all < T

  const int64_t bx = (MODE == kAttn && a.x_period > 0) ? b % a.x_period : b;
  const int64_t by = (MODE == kAttn && a.y_period > 0) ? b % a.y_period : b;
  const int64_t bv = (MODE == kAttn && a.v_period > 0) ? b % a.v_period : b;
  const bf16_t* xg = a.x + bx * a.x_sb + head * 64;
  const bf16_t* yg = a.y + by * a.y_sb + head * 64;
  constexpr bool bounded = (MODE == kAttn || MODE == kLse) && OPT;
  constexpr bool hi_lo = (MODE == kCredit) && OPT;

  bf16x8 xf[OG][4];
#pragma unroll
  for (int og = 0; og < OG; ++og)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int o = wave_live ? ow + og * 32 + col : 0;
      xf[og][kk] = *(const bf16x8*)(xg + (int64_t)o * a.x_st + kk * 16 + half * 8);
    }

  bf16x8 hf[MODE == kCenter ? OG : 1][4];  // kCenter: hub fragments, laid out like xf
  if constexpr (MODE == kCenter) {
    const bf16_t* hg = a.hub + b * a.x_sb + head * 64;
#pragma unroll
    for (int og = 0; og < OG; ++og)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int o = wave_live ? ow + og * 32 + col : 0;
        hf[og][kk] = *(const bf16x8*)(hg + (int64_t)o * a.x_st + kk * 16 + half * 8);
      }
  }

  f32x16 o_acc[OG][2];
#pragma unroll
  for (int og = 0; og < OG; ++og)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o_acc[og][t][r] = 0.f;
  float m_run[OG], l_run[OG], c_run[OG];
#pragma unroll
  for (int og = 0; og < OG; ++og) { m_run[og] = -INFINITY; l_run[og] = 0.f; c_run[og] = 0.f; }
  const float qk_scale = 0.125f * kLog2e;
  if constexpr (bounded) {
    // The bounded softmax's scale log2(e) / 8 goes into the x fragments (one more bf16 rounding of q), so each
    // weight is one exp2 of the MFMA's output.
#pragma unroll
    for (int og = 0; og < OG; ++og)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int j = 0; j < 8; ++j) xf[og][kk][j] = (__bf16)((float)xf[og][kk][j] * qk_scale);
  }

  int i_begin, i_end;  // input range of the whole workgroup [i_begin, i_end)
  if (MODE == kCredit) {
    i_begin = o0;
    i_end = min(T, o0 + kBO + W);
  } else {
    i_begin = max(0, o0 - W);
    i_end = min(T, o0 + kBO);
  }
  i_begin = i_begin / kFlashBI * kFlashBI;

  const float* lse_in = (MODE == kCredit) ? a.lse_in + ((int64_t)b * a.heads + head) * T : nullptr;

  // Tile loads through buffer resources over this row's inputs: per-lane offsets are fixed, the tile's first input
  // goes in the scalar offset, and inputs past T read as zeros.
  constexpr bool kVRows = (MODE == kCenter || MODE == kAttn);
  constexpr int kVElt = (MODE == kCredit) ? 4 : 2;  // bytes per value element
  const __amdgpu_buffer_rsrc_t y_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)yg, 0, (int)(((int64_t)(T - 1) * a.y_st + 64) * 2), 0x00020000);
  const int64_t v_row = (MODE == kCredit && a.v_div > 1) ? (b / a.v_div) * a.v_sb + (b % a.v_div) * 64
                                                          : bv * a.v_sb + head * 64;
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const char*)a.v + v_row * kVElt), 0,
      (MODE == kLse) ? 0 : (int)(((int64_t)(T - 1) * a.v_st + 64) * kVElt), 0x00020000);
  const int y_step = (int)a.y_st * 2, v_step = (int)a.v_st * kVElt;  // bytes per input
  // y tiles (and the bf16 value tiles of kAttn and kCenter) go straight to LDS: load j of wave w fills tile rows
  // 8 (2 w + j) .. + 7, lane l the 16-byte slot l & 7 of row 8 (2 w + j) + (l >> 3), so it fetches the chunk that
  // the row's swizzle puts in that slot. kCredit's fp32 values (4 16-byte chunks per thread) and the LSE values go
  // through registers, converted on the way to LDS.
  constexpr bool kDmaV = kVRows;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  int y_dvo[2], v_dvo[2], v_vo[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = (wv * 2 + j) * 8 + (lane >> 3), chunk = (lane & 7) ^ ((row >> 1) & 7);
    y_dvo[j] = (row * (int)a.y_st + chunk * 8) * 2;
    // kAttn's values in vt_slot's layout (16-byte slot c ^ 2 (row & 3) holds chunk c), kCenter's like y
    const int vchunk = (MODE == kAttn) ? (lane & 7) ^ ((row & 3) << 1) : chunk;
    v_dvo[j] = (row * (int)a.v_st + vchunk * 8) * 2;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) v_vo[k] = (((tid + k * 256) >> 4) * (int)a.v_st + ((tid + k * 256) & 15) * 4) * kVElt;
  auto dma = [&](int i0, int st) {
#pragma unroll
    for (int j = 0; j < 2; ++j) flash_dma16(y_rsrc, &ys[st][(wv * 2 + j) * 512], y_dvo[j], i0 * y_step);
    if constexpr (kDmaV) {
#pragma unroll
      for (int j = 0; j < 2; ++j) flash_dma16(v_rsrc, &vt_hi[st][(wv * 2 + j) * 512], v_dvo[j], i0 * v_step);
    }
  };
  auto load = [&](int i0, FlashStage<MODE>& st) {
    if constexpr (MODE == kCredit) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        st.v[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(v_rsrc, v_vo[k], i0 * v_step, 0));
      st.lse = (tid < 64) ? lse_in[i0 + tid] : 0.f;
    }
  };
  auto store = [&](int s, const FlashStage<MODE>& st) {
    if constexpr (MODE == kCredit) {
      // row-major like the kAttn values: 4 channels of row i as bf16 high and low parts, 8 bytes each
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int v = tid + k * 256, row = v >> 4, c4 = v & 15;
        uint32_t hi[2], lo[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float f0 = st.v[k][2 * j], f1 = st.v[k][2 * j + 1];
          hi[j] = pack_bf16x2(f0, f1);
          if constexpr (hi_lo) lo[j] = pack_bf16x2(f0 - bf16_lo(hi[j]), f1 - bf16_hi(hi[j]));
        }
        const int at = vt_slot(row, c4);
        *(u32x2*)(&vt_hi[s][at]) = u32x2{hi[0], hi[1]};
        if constexpr (hi_lo) *(u32x2*)(&vt_lo[s][at]) = u32x2{lo[0], lo[1]};
      }
      if (tid < 64) lse_s[s][tid] = st.lse * kLog2e;  // staged in log2 units
    }
  };

  FlashStage<MODE> stage;
  dma(i_begin, 0);
  load(i_begin, stage);
  store(0, stage);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();
  // The x (and hub) fragments are loop-invariant registers whose loads may still be in flight here. Each iteration
  // issues the next tile's loads before its first MFMA, and the wait counts the compiler puts in front of those MFMAs
  // are sized for the first iteration; they would then wait for this iteration's tile loads every time. Taking the
  // fragments here makes them resident before the loop, so the loop's MFMAs carry no load waits.
#pragma unroll
  for (int og = 0; og < OG; ++og)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      asm volatile("" ::"v"(xf[og][kk]));
      if constexpr (MODE == kCenter) asm volatile("" ::"v"(hf[og][kk]));
    }

  // One input tile on LDS stage s (a compile-time constant: the loop below runs two tiles per trip, so every LDS
  // address is a register plus a constant).
  auto input_tile = [&](int i0, auto stage_c) __attribute__((always_inline)) {
    constexpr int s = decltype(stage_c)::value;
    // after the first tile nothing counted by vmcnt is in flight here (each tile ends with vmcnt(0)); at the first,
    // this retires what the prologue left (spill stores), so that no wait inside the tile is for them
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    const bool more = i0 + kFlashBI < i_end;
    if (more) {
      dma(i0 + kFlashBI, s ^ 1);
      load(i0 + kFlashBI, stage);
    }

    // per output group: any valid pair in this tile, and no pair masked
    bool any[OG], full[OG];
    bool any_og = false;
#pragma unroll
    for (int og = 0; og < OG; ++og) {
      const int g0 = ow + og * 32;
      if (MODE == kCredit) {
        any[og] = wave_live && (i0 + kFlashBI - 1 >= g0) && (i0 <= g0 + 31 + W);
        full[og] = (i0 >= g0 + 31) && (i0 + kFlashBI - 1 <= g0 + W);
      } else {
        any[og] = wave_live && (i0 <= g0 + 31) && (i0 + kFlashBI - 1 >= g0 - W);
        full[og] = (i0 + kFlashBI - 1 <= g0) && (i0 >= g0 + 31 - W);
      }
      any_og = any_og || any[og];
    }

    if (any_og) {
      // ---- S^T = Y X^T for both output groups; each y fragment is read once ----
      f32x16 sc[OG][2];
      f32x16 s2[MODE == kCenter ? OG : 1][2];  // kCenter: value scores v_i . hub_o
#pragma unroll
      for (int og = 0; og < OG; ++og)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) sc[og][t][r] = 0.f;
      if constexpr (MODE == kCenter) {
#pragma unroll
        for (int og = 0; og < OG; ++og)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) s2[og][t][r] = 0.f;
      }
      if constexpr (MODE == kAttn && OG == 1) {
        // the 8 y fragments through a ring of 4: each read is issued 4 MFMAs before the MFMA that takes it
        bf16x8 yfr[8];
        auto yread = [&](int q) {
          const int row = (q >> 2) * 32 + col;
          return *(const bf16x8*)(&ys[s][row * 64 + ((((q & 3) * 2 + half) ^ ((row >> 1) & 7)) * 8)]);
        };
#pragma unroll
        for (int q = 0; q < 4; ++q) yfr[q] = yread(q);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          sc[0][q >> 2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(yfr[q], xf[0][q & 3], sc[0][q >> 2], 0, 0, 0);
          if (q + 4 < 8) yfr[q + 4] = yread(q + 4);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // 4 LDS reads, then (MFMA, LDS read) x 4, 4 MFMAs
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      } else
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int row = t * 32 + col;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int at = row * 64 + (((kk * 2 + half) ^ ((row >> 1) & 7)) * 8);
          const bf16x8 yf = *(const bf16x8*)(&ys[s][at]);
#pragma unroll
          for (int og = 0; og < OG; ++og)
            if (any[og]) sc[og][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(yf, xf[og][kk], sc[og][t], 0, 0, 0);
          if constexpr (MODE == kCenter) {
            const bf16x8 vf = *(const bf16x8*)(&vt_hi[s][at]);
#pragma unroll
            for (int og = 0; og < OG; ++og)
              if (any[og]) s2[og][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, hf[og][kk], s2[og][t], 0, 0, 0);
          }
        }
      }

      // ---- probabilities: masked pairs of a partial tile get -inf first, so exp2 runs unconditionally ----
#pragma unroll
      for (int og = 0; og < OG; ++og) {
        if (!any[og]) continue;
        const int my_o = ow + og * 32 + col;
        if (!full[og]) {
          // input i = i0 + 4 half + c with c = 32 t + 8 (r / 4) + r % 4 fixed per register, so the lag is base - c
          // (kCredit: c - base) and 0 <= lag <= W is one unsigned compare
          const int base = my_o - (i0 + half * 4);
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int c = t * 32 + (r >> 2) * 8 + (r & 3);
              const uint32_t lag = (uint32_t)((MODE == kCredit) ? c - base : base - c);
              sc[og][t][r] = lag <= (uint32_t)W ? sc[og][t][r] : -INFINITY;
            }
        }
        if (MODE == kCredit) {
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int il = t * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
              sc[og][t][r] = fast_exp2(fmaf(sc[og][t][r], qk_scale, -lse_s[s][il]));
            }
        } else if (bounded) {
          float ls = 0.f;
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float p = fast_exp2(sc[og][t][r]);  // the scores carry the scale (x fragments above)
              sc[og][t][r] = p;
              ls += p;
            }
          l_run[og] += ls;
        } else {
          // the maximum of the raw scores, scaled once (the scale is positive and rounding is monotonic, so this is
          // the maximum of the scaled scores); each weight is then one fma and one exp2
          float mt = -INFINITY;
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[og][t][r]);
          mt = fmaxf(mt, lane_xor32(mt, lane)) * qk_scale;
          const float m_new = fmaxf(m_run[og], mt);
          const float m_safe = (m_new == -INFINITY) ? 0.f : m_new;
          const float corr = fast_exp2(m_run[og] - m_safe);
          float ls = 0.f, cs = 0.f;
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float p = fast_exp2(fmaf(sc[og][t][r], qk_scale, -m_safe));
              sc[og][t][r] = p;
              ls += p;
              if constexpr (MODE == kCenter) cs = fmaf(p, s2[og][t][r], cs);
            }
          l_run[og] = l_run[og] * corr + ls;
          if constexpr (MODE == kCenter) c_run[og] = c_run[og] * corr + cs;
          m_run[og] = m_new;
          if (MODE == kAttn) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int r = 0; r < 16; ++r) o_acc[og][t][r] *= corr;
          }
        }
      }

      // ---- O^T += V^T P^T: 4 k-steps of 16 inputs, 2 tiles of 32 channels; V^T fragments shared by both groups ----
      if constexpr (MODE == kAttn && OG == 1) {
        // the 8 V^T fragments (2 transposing reads each) through a ring of 4, in the order of the loop below
        bf16x8 pf[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int sp = 0; sp < 2; ++sp)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) pf[t][sp][jj] = (__bf16)sc[0][t][sp * 8 + jj];
        const int grp = lane >> 4;
        auto vread = [&](int q) {  // q = 4 t + 2 sp + dt
          const int base = (q >> 2) * 32 + ((q >> 1) & 1) * 16;
          const int d0 = (q & 1) * 32 + 16 * (grp & 1) + 4 * (lane & 3);
          const int i_a = base + 4 * (grp >> 1) + ((lane >> 2) & 3), i_b = i_a + 8;
          const int at_a = vt_slot(i_a, d0 >> 2), at_b = vt_slot(i_b, d0 >> 2);
          const v4s ra = ds_read_tr16(&vt_hi[s][at_a]), rb = ds_read_tr16(&vt_hi[s][at_b]);
          return __builtin_bit_cast(bf16x8, s16x8{ra[0], ra[1], ra[2], ra[3], rb[0], rb[1], rb[2], rb[3]});
        };
        bf16x8 vfr[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) vfr[q] = vread(q);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          o_acc[0][q & 1] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[q], pf[q >> 2][(q >> 1) & 1], o_acc[0][q & 1], 0, 0, 0);
          if (q + 4 < 8) vfr[q + 4] = vread(q + 4);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // 8 LDS reads, then (MFMA, 2 LDS reads) x 4, 4 MFMAs
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      } else if (MODE == kAttn || MODE == kCredit) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int sp = 0; sp < 2; ++sp) {
            bf16x8 pf[OG];
#pragma unroll
            for (int og = 0; og < OG; ++og)
#pragma unroll
              for (int jj = 0; jj < 8; ++jj) pf[og][jj] = (__bf16)sc[og][t][sp * 8 + jj];
            const int base = t * 32 + sp * 16;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
              // Values are rows [input][channel] in LDS; two transposing reads give this lane channel d at the 8 inputs
              // of its k slots (ds_read_b64_tr_b16: in each 16-lane group, lane j gets element j % 4 of the 8-byte
              // pieces read by lanes j / 4 + 4 s, s = 0..3; lane a + 4 s reads channels d0 + 4 a .. of input s).
              const int grp = lane >> 4;
              const int d0 = dt * 32 + 16 * (grp & 1) + 4 * (lane & 3);
              const int i_a = base + 4 * (grp >> 1) + ((lane >> 2) & 3), i_b = i_a + 8;
              // the conflict-free layout of vt_slot (kAttn's values, staged by direct-to-LDS loads, too)
              const int at_a = (MODE == kCredit || MODE == kAttn) ? vt_slot(i_a, d0 >> 2)
                                                 : i_a * 64 + (((d0 >> 3) ^ ((i_a >> 1) & 7)) * 8) + (d0 & 7);
              const int at_b = (MODE == kCredit || MODE == kAttn) ? vt_slot(i_b, d0 >> 2)
                                                 : i_b * 64 + (((d0 >> 3) ^ ((i_b >> 1) & 7)) * 8) + (d0 & 7);
              const v4s ra = ds_read_tr16(&vt_hi[s][at_a]), rb = ds_read_tr16(&vt_hi[s][at_b]);
              const bf16x8 vf = __builtin_bit_cast(bf16x8, s16x8{ra[0], ra[1], ra[2], ra[3], rb[0], rb[1], rb[2], rb[3]});
#pragma unroll
              for (int og = 0; og < OG; ++og)
                if (any[og]) o_acc[og][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[og], o_acc[og][dt], 0, 0, 0);
              if constexpr (hi_lo) {
                const v4s ga = ds_read_tr16(&vt_lo[s][at_a]), gb = ds_read_tr16(&vt_lo[s][at_b]);
                const bf16x8 lf = __builtin_bit_cast(bf16x8, s16x8{ga[0], ga[1], ga[2], ga[3], gb[0], gb[1], gb[2], gb[3]});
#pragma unroll
                for (int og = 0; og < OG; ++og)
                  if (any[og]) o_acc[og][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lf, pf[og], o_acc[og][dt], 0, 0, 0);
              }
            }
          }
      }
    }

    if (more) store(s ^ 1, stage);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // the next tile has landed in LDS
    __syncthreads();
  };
  for (int i0 = i_begin; i0 < i_end; i0 += 2 * kFlashBI) {
    input_tile(i0, std::integral_constant<int, 0>{});
    if (i0 + kFlashBI >= i_end) break;
    input_tile(i0 + kFlashBI, std::integral_constant<int, 1>{});
  }

  if (!wave_live) return;
  // ---- epilogue ----
#pragma unroll
  for (int og = 0; og < OG; ++og) {
    const int my_o = ow + og * 32 + col;
    if (MODE == kAttn || MODE == kLse || MODE == kCenter) {
      const float l_tot = l_run[og] + lane_xor32(l_run[og], lane);
      const float mref = bounded ? 0.f : m_run[og];
      const float lse = (mref + log2f(l_tot)) * (1.0f / kLog2e);
      if (a.lse_out && half == 0) a.lse_out[((int64_t)b * a.heads + head) * T + my_o] = lse;
      if constexpr (MODE == kCenter) {
        const float c_tot = c_run[og] + lane_xor32(c_run[og], lane);
        if (half == 0) a.center_out[((int64_t)b * a.heads + head) * T + my_o] = c_tot / l_tot;
      }
      if (MODE == kAttn) {
        const float inv = 1.0f / l_tot;
        bf16_t* og_ptr = (bf16_t*)a.out + b * a.o_sb + (int64_t)my_o * a.o_st + head * 64;
        // One wave's 32 x 64 output tile in the input-tile LDS, free after the loop's last barrier: 4 waves x 4 KB
        static_assert(4 * 32 * 64 <= 2 * 64 * 64, "4 waves' staged tiles fit the input-tile LDS");
        bf16_t* y_stage = &ys[0][0] + wave * 2048;
        float dot = 0.f;
        const float* bv = nullptr;
        if (a.xb_out) {
          const int32_t xr = a.xb_row[b];
          bv = a.xb_vec + ((uint32_t)xr < (uint64_t)a.xb_rows ? (int64_t)xr : 0) * a.xb_stride + head * 64;
        }
        const bool jit = a.jit_sigma != 0.f;
        const uint32_t jrow = jit ? (uint32_t)((int64_t)a.jit_seq[b] * T + my_o) : 0u;
        const uint32_t jdraw = jit ? (uint32_t)(a.jit_draw0 + b / a.jit_n_seq) : 0u;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d = dt * 32 + g * 8 + half * 4;
            float jz[4] = {0.f, 0.f, 0.f, 0.f};
            if (jit) {
              dust_noise_quad(a.jit_seed, jdraw, a.jit_site, jrow, (uint32_t)(a.heads * 16), (uint32_t)((head * 64 + d) / 4),
                              jz);
#pragma unroll
              for (int j = 0; j < 4; ++j) jz[j] *= a.jit_sigma;
            }
            uint32_t e[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              e[j] = pack_bf16x2(o_acc[og][dt][g * 4 + 2 * j] * inv + jz[2 * j],
                                 o_acc[og][dt][g * 4 + 2 * j + 1] * inv + jz[2 * j + 1]);
              if (bv) dot += bf16_lo(e[j]) * bv[d + 2 * j] + bf16_hi(e[j]) * bv[d + 2 * j + 1];
            }
            if constexpr (OG == 1) {  // staged: row col of the wave's 32 x 64 tile, 16-byte unit swizzled by row
              const int u = (dt * 4 + g) ^ ((col >> 1) & 7);
              *(u32x2*)(y_stage + col * 64 + u * 8 + half * 4) = u32x2{e[0], e[1]};
            } else {
              *(u32x2*)(og_ptr + d) = u32x2{e[0], e[1]};
            }
          }
        if constexpr (OG == 1) {
          // The staged tile leaves as whole 128-byte rows: 8 rows per store instruction, non-temporal (attn_proj
          // reads y after it has left the caches). Only this wave's lanes touch its staging slice.
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int r = k * 8 + (lane >> 3), u = lane & 7;
            const u32x4 val = *(const u32x4*)(y_stage + r * 64 + ((u ^ ((r >> 1) & 7)) * 8));
            __builtin_nontemporal_store(
                val, (u32x4*)((bf16_t*)a.out + b * a.o_sb + (int64_t)(ow + r) * a.o_st + head * 64 + u * 8));
          }
        }
        if (a.xb_out) {
          dot += lane_xor32(dot, lane);
          if (half == 0) a.xb_out[(b * T + my_o) * a.heads + head] = dot;
        }
      }
    } else {
      const int64_t o_div = a.o_div > 1 ? a.o_div : 1;
      const int64_t o_row = a.o_map ? (int64_t)a.o_map[b / o_div] : b / o_div;
      float* og_ptr = (float*)a.out + o_row * a.o_sb + (b % o_div) * 64 + (int64_t)my_o * a.o_st + head * 64;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = dt * 32 + g * 8 + half * 4;
          *(f32x4*)(og_ptr + d) =
              f32x4{o_acc[og][dt][g * 4], o_acc[og][dt][g * 4 + 1], o_acc[og][dt][g * 4 + 2], o_acc[og][dt][g * 4 + 3]};
        }
    }
  }
}

}  // namespace noise

namespace noise {

// One launch of the flash kernel over `batch` x `heads` rows of T tokens (T % 128 == 0).
template <int MODE, bool OPT, int OG>
inline hipError_t launch_flash(const FlashArgs& a, int64_t batch, int heads, hipStream_t stream) {
  constexpr int kBO = FlashTile<OG>::BO;
  hipLaunchKernelGGL((window_flash_kernel<MODE, OPT, OG>), dim3((unsigned)((a.T + kBO - 1) / kBO), (unsigned)heads,
                     (unsigned)batch), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace noise
