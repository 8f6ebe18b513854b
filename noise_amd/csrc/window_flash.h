// Windowed causal flash kernel for head_dim 64 on gfx950, shared by three passes:
//
//   kAttn   out_o = sum_i softmax_i(x_o . y_i / 8) v_i over 0 <= o - i <= W   (attention forward; x = q, y = k)
//           utils/model.py:17-31
//   kLse    lse_o = log sum_i exp(x_o . y_i / 8) over the same window          (credit LSE pass; x = q, y = k)
//           train/speedrun/moment_kernels.py:79-110
//   kCredit out_o = sum_i exp(x_o . y_i / 8 - lse_i) v_i over 0 <= i - o <= W  (credit value pass; x = k, y = q,
//           v = the fp32 source as bf16 high (+ low) parts)  train/speedrun/moment_kernels.py:612-661
//
// A workgroup owns 128 outputs of one (batch, head) row: 4 waves x 32 outputs. Inputs stream through LDS in tiles of
// 64. Scores are computed transposed, S^T[i, o] = y_i . x_o (v_mfma_f32_32x32x16_bf16, y from LDS as the A operand,
// x in registers as the B operand), because the accumulator layout of S^T (lane = output column l%32, registers =
// 16 inputs) is exactly the B-operand layout of O^T[d, o] += V^T[d, i] P^T[i, o]: the probabilities go from the
// score registers to the value MFMA without an LDS round trip. V^T is staged transposed in LDS. Softmax statistics
// are per lane (one output per lane, the other half of the inputs in lane ^ 32).
#pragma once

#include "common.h"

namespace noise {

enum FlashMode { kAttn = 0, kLse = 1, kCredit = 2 };

struct FlashArgs {
  const bf16_t* x;  // output-side vectors [batch, T, heads, 64] with strides below
  const bf16_t* y;  // input-side vectors
  const void* v;    // values: bf16 (kAttn) or fp32 (kCredit)
  int64_t x_sb, x_st, y_sb, y_st, v_sb, v_st;  // strides (elements) of batch and token; head h at +64 h
  const float* lse_in;  // kCredit: [batch * heads, T]
  void* out;            // kAttn: bf16 [batch, T, heads*64] (strides o_sb, o_st); kCredit: fp32 likewise
  int64_t o_sb, o_st;
  float* lse_out;       // kAttn / kLse: [batch * heads, T] (optional for kAttn)
  float* xb_out;        // kAttn (optional): [batch, T, heads] = out_o . xb_vec[h*64 ..] (rank-1 partial dots)
  const float* xb_vec;  // kAttn: per-batch vector base, batch b uses xb_vec + xb_row[b] * xb_stride
  const int32_t* xb_row;
  int64_t xb_stride;
  int32_t heads, T, window, hi_lo;
};

constexpr int kFlashBO = 128, kFlashBI = 64;
constexpr float kLog2e = 1.4426950408889634f;

// LDS: y tile [64][64] bf16 (8 KB), V^T hi [64][64] (8 KB), V^T lo (8 KB), lse tile [64] fp32.
constexpr int kFlashLds = 3 * 64 * 64 * 2 + 64 * 4;

__device__ __forceinline__ int vt_swz(int d, int chunk) { return chunk ^ ((d >> 1) & 15); }  // 8-byte chunks

template <int MODE>
__global__ __launch_bounds__(256) void window_flash_kernel(FlashArgs a) {
  __shared__ __align__(16) unsigned char smem[kFlashLds];
  bf16_t* ys = (bf16_t*)smem;
  bf16_t* vt_hi = ys + 64 * 64;
  bf16_t* vt_lo = vt_hi + 64 * 64;
  float* lse_s = (float*)(vt_lo + 64 * 64);

  const int T = a.T, W = a.window;
  const int n_tiles = T / kFlashBO;
  // heaviest output tiles first (kAttn / kLse: late outputs see the most inputs; kCredit: early ones)
  const int tile = (MODE == kCredit) ? (int)blockIdx.x : n_tiles - 1 - (int)blockIdx.x;
  const int head = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int o0 = tile * kFlashBO;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, col = lane & 31;
  const int ow = o0 + wave * 32;  // this wave's first output
  const int my_o = ow + col;

  const bf16_t* xg = a.x + b * a.x_sb + head * 64;
  const bf16_t* yg = a.y + b * a.y_sb + head * 64;

  // x_o for this lane's output as four B-operand fragments (dims 16 kk + 8 half .. +7)
  bf16x8 xf[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) xf[kk] = *(const bf16x8*)(xg + (int64_t)my_o * a.x_st + kk * 16 + half * 8);

  f32x16 o_acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float qk_scale = 0.125f * kLog2e;

  int i_begin, i_end;  // input range of the whole workgroup [i_begin, i_end)
  if (MODE == kCredit) {
    i_begin = o0;
    i_end = min(T, o0 + kFlashBO + W);
  } else {
    i_begin = max(0, o0 - W);
    i_end = o0 + kFlashBO;
  }
  i_begin = i_begin / kFlashBI * kFlashBI;

  const float* lse_in = (MODE == kCredit) ? a.lse_in + ((int64_t)b * a.heads + head) * T : nullptr;

  for (int i0 = i_begin; i0 < i_end; i0 += kFlashBI) {
    // ---- stage y tile (swizzled rows of 8 chunks) and V^T ----
    __syncthreads();
#pragma unroll
    for (int rep = 0; rep < 2; ++rep) {
      const int v = threadIdx.x + rep * 256;
      const int row = v >> 3, chunk = v & 7;
      const u32x4 val = *(const u32x4*)(yg + (int64_t)(i0 + row) * a.y_st + chunk * 8);
      *(u32x4*)(ys + row * 64 + ((chunk ^ (row & 7)) * 8)) = val;
    }
    if (MODE == kAttn) {
      const bf16_t* vg = (const bf16_t*)a.v + b * a.v_sb + head * 64;
#pragma unroll
      for (int rep = 0; rep < 2; ++rep) {
        const int v = threadIdx.x + rep * 256;
        const int row = v >> 3, d0 = (v & 7) * 8;  // input row, first of 8 dims
        const u32x4 val = *(const u32x4*)(vg + (int64_t)(i0 + row) * a.v_st + d0);
        const bf16_t* e = (const bf16_t*)&val;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int d = d0 + j;
          vt_hi[d * 64 + vt_swz(d, row >> 2) * 4 + (row & 3)] = e[j];
        }
      }
    } else if (MODE == kCredit) {
      const float* vg = (const float*)a.v + b * a.v_sb + head * 64;
#pragma unroll
      for (int rep = 0; rep < 4; ++rep) {
        const int v = threadIdx.x + rep * 256;
        const int row = v >> 4, d0 = (v & 15) * 4;
        const f32x4 val = *(const f32x4*)(vg + (int64_t)(i0 + row) * a.v_st + d0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = d0 + j;
          const bf16_t hi = f32_to_bf16(val[j]);
          const int at = d * 64 + vt_swz(d, row >> 2) * 4 + (row & 3);
          vt_hi[at] = hi;
          vt_lo[at] = f32_to_bf16(val[j] - bf16_to_f32(hi));
        }
      }
      if (threadIdx.x < 64) lse_s[threadIdx.x] = (i0 + threadIdx.x < T) ? lse_in[i0 + threadIdx.x] : 0.f;
    }
    __syncthreads();

    // ---- per-wave skip of tiles with no valid pair ----
    bool any, full;
    if (MODE == kCredit) {
      any = (i0 + kFlashBI - 1 >= ow) && (i0 <= ow + 31 + W);
      full = (i0 >= ow + 31) && (i0 + kFlashBI - 1 <= ow + W);
    } else {
      any = (i0 <= ow + 31) && (i0 + kFlashBI - 1 >= ow - W);
      full = (i0 + kFlashBI - 1 <= ow) && (i0 >= ow + 31 - W);
    }
    if (!any) continue;

    // ---- S^T = Y X^T: two 32-input tiles ----
    f32x16 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
      const int row = t * 32 + col;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8 yf = *(const bf16x8*)(ys + row * 64 + (((kk * 2 + half) ^ (row & 7)) * 8));
        s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(yf, xf[kk], s[t], 0, 0, 0);
      }
    }

    // ---- probabilities (in place, as base-2 logits then weights) ----
    if (MODE == kCredit) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int il = t * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
          const int i = i0 + il;
          const bool ok = full || ((i - my_o) >= 0 && (i - my_o) <= W && i < T);
          const float e = s[t][r] * qk_scale - lse_s[il] * kLog2e;
          s[t][r] = ok ? fast_exp2(e) : 0.f;
        }
    } else {
      float mt = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = i0 + t * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
          const bool ok = full || ((my_o - i) >= 0 && (my_o - i) <= W);
          const float e = ok ? s[t][r] * qk_scale : -INFINITY;
          s[t][r] = e;
          mt = fmaxf(mt, e);
        }
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const float m_new = fmaxf(m_run, mt);
      const float m_safe = (m_new == -INFINITY) ? 0.f : m_new;
      const float corr = fast_exp2(m_run - m_safe);
      float ls = 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(s[t][r] - m_safe);
          s[t][r] = p;
          ls += p;
        }
      l_run = l_run * corr + ls;
      m_run = m_new;
      if (MODE == kAttn) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) o_acc[t][r] *= corr;
      }
    }

    // ---- O^T += V^T P^T: 4 k-steps of 16 inputs, 2 tiles of 32 dims ----
    if (MODE != kLse) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int sp = 0; sp < 2; ++sp) {
          bf16x8 pf;
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) pf[jj] = (__bf16)s[t][sp * 8 + jj];
          const int base = t * 32 + sp * 16;
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) {
            const int d = dt * 32 + col;
            const int c0 = (base + 4 * half) >> 2, c1 = (base + 8 + 4 * half) >> 2;
            const u32x2 lo4 = *(const u32x2*)(vt_hi + d * 64 + vt_swz(d, c0) * 4);
            const u32x2 hi4 = *(const u32x2*)(vt_hi + d * 64 + vt_swz(d, c1) * 4);
            const u32x4 packed = {lo4[0], lo4[1], hi4[0], hi4[1]};
            o_acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, packed), pf, o_acc[dt], 0, 0, 0);
            if (MODE == kCredit && a.hi_lo) {
              const u32x2 l0 = *(const u32x2*)(vt_lo + d * 64 + vt_swz(d, c0) * 4);
              const u32x2 l1 = *(const u32x2*)(vt_lo + d * 64 + vt_swz(d, c1) * 4);
              const u32x4 pl = {l0[0], l0[1], l1[0], l1[1]};
              o_acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, pl), pf, o_acc[dt], 0, 0, 0);
            }
          }
        }
    }
  }

  // ---- epilogue ----
  if (MODE == kAttn || MODE == kLse) {
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float lse = (m_run + log2f(l_tot)) * (1.0f / kLog2e);
    if (a.lse_out && half == 0) a.lse_out[((int64_t)b * a.heads + head) * T + my_o] = lse;
    if (MODE == kAttn) {
      const float inv = 1.0f / l_tot;
      bf16_t* og = (bf16_t*)a.out + b * a.o_sb + (int64_t)my_o * a.o_st + head * 64;
      float dot = 0.f;
      const float* bv = a.xb_out ? a.xb_vec + (int64_t)a.xb_row[b] * a.xb_stride + head * 64 : nullptr;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = dt * 32 + g * 8 + half * 4;
          bf16_t e[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            e[j] = f32_to_bf16(o_acc[dt][g * 4 + j] * inv);
            if (bv) dot += bf16_to_f32(e[j]) * bv[d + j];
          }
          *(u32x2*)(og + d) = u32x2{(uint32_t)e[0] | ((uint32_t)e[1] << 16), (uint32_t)e[2] | ((uint32_t)e[3] << 16)};
        }
      if (a.xb_out) {
        dot += __shfl_xor(dot, 32, 64);
        if (half == 0) a.xb_out[(b * T + my_o) * a.heads + head] = dot;
      }
    }
  } else {
    float* og = (float*)a.out + b * a.o_sb + (int64_t)my_o * a.o_st + head * 64;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = dt * 32 + g * 8 + half * 4;
        *(f32x4*)(og + d) = f32x4{o_acc[dt][g * 4], o_acc[dt][g * 4 + 1], o_acc[dt][g * 4 + 2], o_acc[dt][g * 4 + 3]};
      }
  }
}

}  // namespace noise
