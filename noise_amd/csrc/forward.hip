// The perturbed population forward of the fixed GPT (archive/10M/train/val/eggroll.py:66-103 over
// utils/model.py:193-210), as row kernels + bf16 MFMA GEMMs with population epilogues + the windowed flash kernel.
//
// Rows: member i's token t is row r = i * T + t of every activation (T % 128 == 0). The rank-1 correction
// sign * (x . b) a^T of eggroll.py:56-58 is split between the producer of x, which writes x . b per row (or per-head /
// per-tile partials of it), and the GEMM epilogue, which adds sign * (x . b) * a[col].
#include <math.h>
#include <string.h>

#include "gemm.h"
#include "rng.h"
#include "window_flash.h"

namespace noise {

constexpr float kNormEps = 1.1920928955078125e-07f;  // torch.finfo(torch.float32).eps, F.rms_norm's default

// The lambda mix l_r x + l_0 x0 (eggroll.py:77-79), spelled as one multiply and one fma so that every kernel that forms
// it (the embedding kernel for block 0's input, the projections that recompute that input or mix the next block's)
// rounds it the same way.
__device__ __forceinline__ float lambda_mix(float lr, float l0, float x, float x0) { return fmaf(l0, x0, lr * x); }

// The member tables. A member whose token row is outside [0, n_seq) or whose noise row is outside [0, n_rows) reads
// row 0 of both (so every access stays inside its buffer) and is marked bad: the embedding gives its rows NaN and the
// CE finalization writes NaN for every one of its tokens, so its loss is NaN (the reference's indexing would raise).
struct Members {
  int T;
  const int32_t* seq;   // token row of each member
  const int32_t* row;   // noise row of each member
  const float* sign;    // +-sigma of each member
  const float* noise;   // [n_rows, stride] or NULL (unperturbed)
  int64_t stride;
  const int64_t* tokens;   // [n_seq, T]
  int64_t n_seq, n_rows;
  __device__ __forceinline__ int member(int64_t r) const { return (int)(r / T); }
  __device__ __forceinline__ bool seq_ok(int m) const { return (uint32_t)seq[m] < (uint64_t)n_seq; }
  __device__ __forceinline__ bool row_ok(int m) const { return !noise || (uint32_t)row[m] < (uint64_t)n_rows; }
  __device__ __forceinline__ bool bad(int m) const { return !(seq_ok(m) && row_ok(m)); }
  __device__ __forceinline__ int sq(int m) const { return seq_ok(m) ? seq[m] : 0; }  // the member's token row
  __device__ __forceinline__ const float* nrow(int m) const {
    return noise ? noise + (int64_t)(row_ok(m) ? row[m] : 0) * stride : nullptr;
  }
  __device__ __forceinline__ float sgn(int m) const { return noise ? sign[m] : 0.f; }
  __device__ __forceinline__ int64_t token(int64_t r) const {
    const int m = member(r);
    return tokens[(int64_t)sq(m) * T + (r - (int64_t)m * T)];
  }
};

// Activation jitter of the direct draws (train/val/dust.py:210-233): sigma a added at one site of the entry block.
// Members are (draw, batch row) pairs in draw-major order, so member m is draw draw0 + m / n_seq of batch row seq[m];
// the jitter of (draw, site, token row, 4 channels) comes from the counter stream (rng.h dust_noise_quad).
struct Jitter {
  float sigma;  // 0: no jitter
  uint32_t site;
  uint64_t seed;
  int draw0, n_seq;
  __host__ __device__ __forceinline__ bool on() const { return sigma != 0.f; }
  // sigma a at member row r, channels c .. c + 3 of a site `width` wide
  __device__ __forceinline__ f32x4 quad(const Members& mb, int64_t r, int width, int c) const {
    const int m = mb.member(r);
    const uint32_t row = (uint32_t)((int64_t)mb.sq(m) * mb.T + (r - (int64_t)m * mb.T));
    float z[4];
    dust_noise_quad(seed, (uint32_t)(draw0 + m / n_seq), site, row, (uint32_t)(width / 4), (uint32_t)(c / 4), z);
    return f32x4{sigma * z[0], sigma * z[1], sigma * z[2], sigma * z[3]};
  }
};

// ---------------------------------------------------------------------------------------------------------------
// x0 = norm(wte[tok] + sign a[tok] b [+ the direct draws' jitter])  (eggroll.py:61-63, 74; dust.py:218-220); 8 rows
// per wave, 8 channels per lane. The kernel also forms block 0's input (eggroll.py:77-79, the work mix_norm_kernel does
// for a later first block): x = (l_r + s eps_r) x0 + (l_0 + s eps_0) x0, h = norm(x) in bf16 and the three q/k/v dots
// h . b. x0 itself is written only when asked: a capture, or later mixes that read it instead of recomputing it.
struct EmbedMix {
  float* x;
  bf16_t* h;
  float* xb;  // [M, 4]
  const float* resid_lambdas;
  const float* x0_lambdas;
  int64_t off_resid, off_x0, off_b[3];
  int write_x0;
  int write_x;  // 0: block 0's attn c_proj rebuilds x from x0 itself
};

__global__ __launch_bounds__(256) void embed_kernel(Members mb, const float* __restrict__ wte, int Vp, int64_t off_wte,
                                                    Jitter jit, float* __restrict__ x0, float* __restrict__ x0_inv,
                                                    EmbedMix em, int64_t M) {
  // 8 consecutive rows per wave (M and the member length are multiples of 8, so they belong to one member): lanes
  // 0..7 fetch the rows' tokens and noise scalars together, the member's b vector is read once, and the 8 embedding
  // rows are loaded before any is reduced, so the dependent loads (member table, token, embedding row) overlap.
  const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8;
  if (r0 >= M) return;
  const int lane = threadIdx.x & 63, c0 = lane * 8;
  const int m = mb.member(r0);
  const float* nr = mb.nrow(m);
  const float s = mb.sgn(m);
  int tk = 0, bad = 0;
  float at = 0.f;
  if (lane < 8) {
    const int64_t t = mb.token(r0 + lane);
    bad = t < 0 || t >= Vp || mb.bad(m);
    tk = bad ? 0 : (int)t;
    if (nr) at = s * nr[off_wte + tk];
  }
  float b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) b[j] = nr ? nr[off_wte + Vp + c0 + j] : 0.f;
  float e[8][8], ss[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int tq = lane_val(tk, q);
    const f32x4 w0 = *(const f32x4*)(wte + (int64_t)tq * kD + c0), w1 = *(const f32x4*)(wte + (int64_t)tq * kD + c0 + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) { e[q][j] = w0[j]; e[q][4 + j] = w1[j]; }
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float aq = lane_val(at, q);
    if (nr) {
#pragma unroll
      for (int j = 0; j < 8; ++j) e[q][j] = fmaf(aq, b[j], e[q][j]);  // the mlp_proj epilogue's x0 recompute repeats this
    }
    if (jit.on()) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 z = jit.quad(mb, r0 + q, kD, c0 + 4 * h);
#pragma unroll
        for (int j = 0; j < 4; ++j) e[q][4 * h + j] += z[j];
      }
    }
    ss[q] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss[q] += e[q][j] * e[q][j];
  }
  const float tot = warp_sum8(ss, lane);  // lane l: row (l >> 3) & 7
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float inv = lane_val(bad, q) ? __builtin_nanf("") : rsq_norm(lane_val(tot, 8 * q) * (1.0f / kD) + kNormEps);
    if (lane == q) x0_inv[r0 + q] = inv;
#pragma unroll
    for (int j = 0; j < 8; ++j) e[q][j] *= inv;  // x0
    if (em.write_x0) {
      float* dst = x0 + (r0 + q) * kD + c0;
      *(f32x4*)dst = f32x4{e[q][0], e[q][1], e[q][2], e[q][3]};
      *(f32x4*)(dst + 4) = f32x4{e[q][4], e[q][5], e[q][6], e[q][7]};
    }
  }
  {
    float lr = em.resid_lambdas[0], l0 = em.x0_lambdas[0];
    if (nr) { lr = fmaf(s, nr[em.off_resid], lr); l0 = fmaf(s, nr[em.off_x0], l0); }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
#pragma unroll
      for (int j = 0; j < 8; ++j) e[q][j] = lambda_mix(lr, l0, e[q][j], e[q][j]);  // x
      if (em.write_x) {  // otherwise block 0's attn c_proj rebuilds x from x0 (EpiResidNorm kXBase)
        float* dst = em.x + (r0 + q) * kD + c0;
        *(f32x4*)dst = f32x4{e[q][0], e[q][1], e[q][2], e[q][3]};
        *(f32x4*)(dst + 4) = f32x4{e[q][4], e[q][5], e[q][6], e[q][7]};
      }
      ss[q] = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss[q] += e[q][j] * e[q][j];
    }
    const float tot2 = warp_sum8(ss, lane);
    float d[3][8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float inv = rsq_norm(lane_val(tot2, 8 * q) * (1.0f / kD) + kNormEps);
      u32x4 packed;
#pragma unroll
      for (int j = 0; j < 4; ++j) packed[j] = pack_bf16x2(e[q][2 * j] * inv, e[q][2 * j + 1] * inv);
      *(u32x4*)(em.h + (r0 + q) * kD + c0) = packed;
#pragma unroll
      for (int j = 0; j < 4; ++j) { e[q][2 * j] = bf16_lo(packed[j]); e[q][2 * j + 1] = bf16_hi(packed[j]); }  // h
#pragma unroll
      for (int k = 0; k < 3; ++k) d[k][q] = 0.f;
    }
    if (nr) {
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const f32x4 b0 = *(const f32x4*)(nr + em.off_b[k] + c0), b1 = *(const f32x4*)(nr + em.off_b[k] + c0 + 4);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
#pragma unroll
          for (int j = 0; j < 4; ++j) d[k][q] += e[q][j] * b0[j] + e[q][4 + j] * b1[j];
        }
        const float dt = warp_sum8(d[k], lane);
        if ((lane & 7) == 0) em.xb[(r0 + (lane >> 3)) * 4 + k] = dt;
      }
    } else if (lane < 8) {
#pragma unroll
      for (int k = 0; k < 3; ++k) em.xb[(r0 + lane) * 4 + k] = 0.f;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// [optional lambda mix] x = (l_r + s eps_r) x + (l_0 + s eps_0) x0 (eggroll.py:77-79), then h = norm(x) in bf16, the
// dots h . b_k for up to 3 rank-1 vectors, and the value-embedding gate 2 sigmoid(h[:32] W_g^T + s (h[:32].b_g) a_g)
// (eggroll.py:88). One wave per row.
struct NormArgs {
  float* x;             // [M, 512] fp32 (read; written back when mixing)
  const float* x0;      // [M, 512] (mixing only)
  int mix, first;       // first: x is taken to be x0
  const float* resid_lambdas; const float* x0_lambdas; int layer;
  int64_t off_resid, off_x0;
  bf16_t* h;            // [M, 512]
  int ndot; int64_t off_b[3];  // noise offsets of the b vectors
  float* xb;            // [M, 4]
  const float* w_gate;  // [8, 32] or NULL
  int64_t off_gate;     // noise offset of ve_gate's (a[8] | b[32])
  float* gate;          // [M, 8]
  int64_t M;
};

__global__ __launch_bounds__(256) void mix_norm_kernel(Members mb, NormArgs a) {
  const int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.M) return;
  const int lane = threadIdx.x & 63, c0 = lane * 8;
  const int m = mb.member(r);
  const float* nr = mb.nrow(m);
  const float s = mb.sgn(m);
  float v[8];
  const float* src = a.first ? a.x0 : a.x;
  const f32x4 v0 = *(const f32x4*)(src + r * kD + c0), v1 = *(const f32x4*)(src + r * kD + c0 + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) { v[j] = v0[j]; v[j + 4] = v1[j]; }
  if (a.mix) {
    float lr = a.resid_lambdas[a.layer], l0 = a.x0_lambdas[a.layer];
    if (nr) { lr = fmaf(s, nr[a.off_resid + a.layer], lr); l0 = fmaf(s, nr[a.off_x0 + a.layer], l0); }
    const f32x4 w0 = *(const f32x4*)(a.x0 + r * kD + c0), w1 = *(const f32x4*)(a.x0 + r * kD + c0 + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = lambda_mix(lr, l0, v[j], w0[j]);
      v[j + 4] = lambda_mix(lr, l0, v[j + 4], w1[j]);
    }
    float* dst = a.x + r * kD + c0;
    *(f32x4*)dst = f32x4{v[0], v[1], v[2], v[3]};
    *(f32x4*)(dst + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += v[j] * v[j];
  ss = warp_sum(ss);
  const float inv = rsq_norm(ss * (1.0f / kD) + kNormEps);
  float hv[8];
  u32x4 packed;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    packed[j] = pack_bf16x2(v[2 * j] * inv, v[2 * j + 1] * inv);
    hv[2 * j] = bf16_lo(packed[j]);
    hv[2 * j + 1] = bf16_hi(packed[j]);
  }
  *(u32x4*)(a.h + r * kD + c0) = packed;
  if (nr) {
    for (int k = 0; k < a.ndot; ++k) {
      const float* bv = nr + a.off_b[k] + c0;
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) d += hv[j] * bv[j];
      d = warp_sum(d);
      if (lane == 0) a.xb[r * 4 + k] = d;
    }
  }
  if (a.w_gate) {
    // channels 0..31 live in lanes 0..3
    float g[kH], db = 0.f;
#pragma unroll
    for (int hd = 0; hd < kH; ++hd) {
      float d = 0.f;
      if (lane < 4) {
#pragma unroll
        for (int j = 0; j < 8; ++j) d += hv[j] * a.w_gate[hd * kGateIn + c0 + j];
      }
      g[hd] = d;
    }
    if (nr && lane < 4) {
#pragma unroll
      for (int j = 0; j < 8; ++j) db += hv[j] * nr[a.off_gate + kH + c0 + j];
    }
#pragma unroll
    for (int hd = 0; hd < kH; ++hd) {
      g[hd] += dpp_mov<0xB1>(g[hd]);  // lane ^ 1
      g[hd] += dpp_mov<0x4E>(g[hd]);  // lane ^ 2
    }
    db += dpp_mov<0xB1>(db);
    db += dpp_mov<0x4E>(db);
    if (lane == 0) {
#pragma unroll
      for (int hd = 0; hd < kH; ++hd) {
        float pre = g[hd];
        if (nr) pre += s * db * nr[a.off_gate + hd];
        a.gate[r * kH + hd] = 2.0f / (1.0f + expf(-pre));
      }
    }
  }
}

// gate[r, hd] = 2 sigmoid(h[r, :32] . W_g[hd] + s (h[r, :32] . b_g) a_g[hd]) (eggroll.py:85-89), for a block with
// value embeddings whose h comes from a GEMM epilogue; 8 lanes per row, lane hd of the row computes head hd. The
// channel sums go in chunks of 8 combined pairwise, as in mix_norm_kernel. A workgroup's 32 rows belong to one member
// (T % 128 == 0), so W_g and the member's a_g, b_g are staged in LDS once per workgroup.
__global__ __launch_bounds__(256) void gate_kernel(Members mb, const bf16_t* __restrict__ h,
                                                   const float* __restrict__ w_gate, int64_t off_gate,
                                                   float* __restrict__ gate, int64_t M) {
  static_assert(kH * kGateIn == 256, "one W_g element per thread");
  __shared__ __align__(16) float wg[kH * kGateIn];
  __shared__ __align__(16) float bg[kGateIn];
  __shared__ float ag[kH];
  const int64_t r0 = (int64_t)blockIdx.x * 32;  // < M: the grid has ceil(M / 32) workgroups
  const int m = mb.member(r0);
  const float* nr = mb.nrow(m);
  wg[threadIdx.x] = w_gate[threadIdx.x];
  if (nr && threadIdx.x < kGateIn) bg[threadIdx.x] = nr[off_gate + kH + threadIdx.x];
  if (nr && threadIdx.x < kH) ag[threadIdx.x] = nr[off_gate + threadIdx.x];
  __syncthreads();
  const int64_t r = r0 + (threadIdx.x >> 3);
  if (r >= M) return;
  const int hd = threadIdx.x & 7;
  const float s = mb.sgn(m);
  float g[4], db[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const u32x4 p = *(const u32x4*)(h + r * kD + 8 * c);
    float hv[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) { hv[2 * j] = __uint_as_float(p[j] << 16); hv[2 * j + 1] = __uint_as_float(p[j] & 0xFFFF0000u); }
    const f32x4 w0 = *(const f32x4*)&wg[hd * kGateIn + 8 * c], w1 = *(const f32x4*)&wg[hd * kGateIn + 8 * c + 4];
    const float w[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
    g[c] = 0.f; db[c] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) g[c] += hv[j] * w[j];
    if (nr) {
      const f32x4 b0 = *(const f32x4*)&bg[8 * c], b1 = *(const f32x4*)&bg[8 * c + 4];
      const float bb[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
      for (int j = 0; j < 8; ++j) db[c] += hv[j] * bb[j];
    }
  }
  float pre = (g[0] + g[1]) + (g[2] + g[3]);
  if (nr) pre += s * ((db[0] + db[1]) + (db[2] + db[3])) * ag[hd];
  gate[r * kH + hd] = 2.0f / (1.0f + expf(-pre));
}

// GEMM epilogues. The GEMM hands over one output row per wave: lane l holds columns n0 + 4l .. n0 + 4l + 3 of the
// workgroup's 256-column tile. Noise rows are 16-byte aligned and every parameter slice starts at a multiple of 4.

__device__ __forceinline__ f32x4 ld4(const float* p) { return *(const f32x4*)p; }

// Streaming store of 4 bf16: the GEMM outputs are read next by another kernel, after they have left the caches, so
// the stores are non-temporal.
__device__ __forceinline__ void st_bf16x4(bf16_t* p, f32x4 v) {
  __builtin_nontemporal_store((u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])}), (u32x2*)p);
}

// q|k|v = h W_qkv^T + s (h . b_seg) a_seg (eggroll.py:80-84); on q and k columns then the rotary embedding and the
// per-head RMS norm (utils/model.py:55-58, 93-94: lanes l and l ^ 8 hold the rotary pairs (d, d + 32), 16 lanes a
// head); on v columns the gated value embedding gate * (ve[tok] + s a_ve[tok] b_ve) (eggroll.py:85-89).
struct EpiQKV {
  Members mb;
  bf16_t* out;
  int64_t off[3];     // noise offsets of c_q, c_k, c_v
  const float* xb;    // [M, 4]
  const float* gate;  // [M, 8] or NULL
  const float* ve;    // [Vp, 512] or NULL
  int64_t off_ve;
  int Vp;
  const u32x4* rope;   // [T, 16]: rope_table_kernel's per-lane rotary values
  static constexpr int kRows = kEpiRows;
  struct Wave {
    int row_base, t0, seg, c;
    const float* nr;
    float s, xb, at;
    int tok;
    f32x4 a, b_ve;
  };
  // q / k columns: the row's rotary values from the per-lane table (bf16 pairs: 4 cos, then 4 sin with the rotation's
  // sign); v columns: the row's value-embedding values (fp32 bits) and its gate.
  struct Pre {
    u32x4 w[kEpiRows];
    float g[kEpiRows];
  };
  __device__ __forceinline__ void begin(int row_base, int n0, int lane, int nrows, Wave& w) const {
    const int m = mb.member(row_base);
    w.row_base = row_base;
    w.t0 = row_base - m * mb.T;
    w.seg = n0 >> 9;
    w.c = (n0 & (kD - 1)) + 4 * lane;
    w.nr = mb.nrow(m);
    w.s = mb.sgn(m);
    w.xb = 0.f; w.at = 0.f; w.tok = 0;
    w.a = w.b_ve = f32x4{0.f, 0.f, 0.f, 0.f};
    if (w.nr) {
      w.a = ld4(w.nr + off[w.seg] + w.c);
      if (lane < nrows) w.xb = xb[(int64_t)(row_base + lane) * 4 + w.seg];
    }
    if (w.seg == 2 && ve) {
      const int64_t tk = lane < nrows ? mb.tokens[(int64_t)mb.sq(m) * mb.T + w.t0 + lane] : 0;
      w.tok = (tk < 0 || tk >= Vp) ? 0 : (int)tk;
      if (w.nr) {
        w.at = w.nr[off_ve + w.tok];  // times the sign in ready()
        w.b_ve = ld4(w.nr + off_ve + Vp + w.c);
      }
    }
  }
  __device__ __forceinline__ void ready(Wave& w) const { w.at *= w.s; }
  __device__ __forceinline__ void load(int row0, int, int lane, const Wave& w, Pre& p) const {
    const int i0 = row0 - w.row_base;
    if (w.seg < 2) {
#pragma unroll
      for (int q = 0; q < kEpiRows; ++q) p.w[q] = rope[(w.t0 + i0 + q) * 16 + (lane & 15)];
    } else if (ve) {
#pragma unroll
      for (int q = 0; q < kEpiRows; ++q) {
        p.w[q] = __builtin_bit_cast(u32x4, ld4(ve + (int64_t)lane_val(w.tok, i0 + q) * kD + w.c));
        p.g[q] = gate[(int64_t)(row0 + q) * kH + (w.c >> 6)];
      }
    }
  }
  template <int R>
  __device__ __forceinline__ void rows(int row0, int n0, int, int lane, const Wave& w, const Pre& p,
                                       f32x4 (&v)[R]) const {
    const int i0 = row0 - w.row_base;
    if (w.nr) {
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const float k = lane_val(w.xb, i0 + q);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[q][e] += w.s * k * w.a[e];
      }
    }
    if (w.seg < 2) {
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const float cs[4] = {bf16_lo(p.w[q][0]), bf16_hi(p.w[q][0]), bf16_lo(p.w[q][1]), bf16_hi(p.w[q][1])};
        const float sn[4] = {bf16_lo(p.w[q][2]), bf16_hi(p.w[q][2]), bf16_lo(p.w[q][3]), bf16_hi(p.w[q][3])};
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float other = dpp_mov<0x128>(v[q][e]);  // lane ^ 8: the rotary partner in the head's 16 lanes
          v[q][e] = v[q][e] * cs[e] + other * sn[e];  // sn carries the sign: - on the head's second half
          ss += v[q][e] * v[q][e];
        }
        ss = group_sum8(ss);
        ss += dpp_mov<0x140>(ss);  // the head's 16 lanes
        const float inv = rsq_norm(ss * (1.0f / kHD) + kNormEps);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[q][e] *= inv;
      }
    } else if (ve) {
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const float at = lane_val(w.at, i0 + q);
        const f32x4 e4 = __builtin_bit_cast(f32x4, p.w[q]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[q][e] += p.g[q] * (e4[e] + at * w.b_ve[e]);
      }
    }
#pragma unroll
    for (int q = 0; q < R; ++q) st_bf16x4(out + (int64_t)(row0 + q) * kQKV + n0 + 4 * lane, v[q]);
  }
};

// x += acc + s (sum of the xb partials) a (the residual adds of utils/model.py:118-119); with kMix, then the next
// block's lambda mix x = (l_r + s eps_r) x + (l_0 + s eps_0) x0 (eggroll.py:77-79); x is written back, and
// h = norm(x) in bf16 (utils/model.py:46-47) with the kNDot dots h . b_k of the next linear's rank-1 terms. The tile
// holds whole 512-wide rows (512-column tiles): lane l has columns 4l .. 4l+3 and 256 + 4l .. 256 + 4l + 3. Groups of
// 4 rows keep the x and x0 prefetch small. The rank-1 term is added unconditionally: its a and dot are zero for rows
// without noise. x and h are written with non-temporal stores: neither is read again before it has left the caches.
// kFinal: the last block's c_proj, after which x is not read again: only h and the dots are stored.
// kXBase: block 0's attn c_proj when the embedding kernel stored no x: the residual it adds to is block 0's input
// x = (l_r + s eps_r) x0 + (l_0 + s eps_0) x0, rebuilt from the recomputed x0 (kX0) with embed_kernel's operations, so
// it is bit-identical to the x the embedding kernel would have stored, and 2 KB per row are neither written nor read.
template <bool kMix, int kNDot, bool kJit = false, bool kX0 = false, bool kFinal = false, bool kXBase = false>
struct EpiResidNorm {
  static_assert(!kXBase || (kX0 && !kMix), "block 0's input comes from the recomputed x0, with no mix after it");
  static constexpr int kRows = 4;
  Members mb;
  float* x;             // [M, 512] residual stream, read and written
  const float* xbp;     // [M, nxb] partial dots of this linear's input with its b
  int nxb;
  int64_t off;          // noise offset of this linear's a
  const float* x0;      // [M, 512] (mix only; kX0: recomputed instead)
  // kX0: the mix's x0 recomputed as (wte[tok] + sign a[tok] b) * x0_inv, exactly as embed_kernel forms it, from the
  // embedding row (cache-resident table) instead of a 2 KB HBM read per row
  const float* wte;
  const float* x0_inv;  // [M] embed_kernel's per-row norm scale
  int Vp;
  int64_t off_wte;
  const float* resid_lambdas;
  const float* x0_lambdas;
  int layer;            // the block whose lambdas mix (kXBase: block 0, whose lambdas form its input)
  int64_t off_resid, off_x0;
  bf16_t* h;            // [M, 512]
  int64_t off_b[3];     // noise offsets of the next linear's b vectors (kNDot of them)
  float* xb;            // [M, 4]
  Jitter jit;           // kJit: the direct draws' jitter of this projection's output
  // the partials per row: one per attention head (attn c_proj) or per 256-column tile of c_fc (mlp c_proj)
  static constexpr int kParts = 8;
  static_assert(kH <= kParts && kF / 256 <= kParts, "every caller's partials fit");
  struct Wave {
    int row_base;
    const float* nr;
    float s, d, lr, l0;
    f32x4 a[2];
    u32x2 b[kNDot][2];  // the next linears' b at this lane's columns, as bf16 pairs (the reference's x @ b.to(bf16))
    int tok;         // kX0, by lane: the row's token, its noise scalar sign a[tok] and norm scale
    float at, inv;
    f32x4 bw[2];     // kX0: the embedding's b vector at this lane's columns
    float dp[kParts];  // by lane: the row's partials of this linear's input dot as loaded; ready() sums them into d
  };
  struct Pre {
    f32x4 xv[kRows][2], x0v[kRows][2];
  };
  __device__ __forceinline__ void begin(int row_base, int, int lane, int nrows, Wave& w) const {
    const int m = mb.member(row_base);
    w.row_base = row_base;
    w.nr = mb.nrow(m);
    w.s = mb.sgn(m);
    w.d = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      w.a[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < kNDot; ++k) w.b[k][hh] = u32x2{0u, 0u};
    }
#pragma unroll
    for (int p = 0; p < kParts; ++p) w.dp[p] = 0.f;
    if (w.nr) {
      if (lane < nrows) {
#pragma unroll
        for (int p = 0; p < kParts; ++p)
          if (p < nxb) w.dp[p] = xbp[(int64_t)(row_base + lane) * nxb + p];
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        w.a[hh] = ld4(w.nr + off + hh * 256 + 4 * lane);
#pragma unroll
        for (int k = 0; k < kNDot; ++k) {
          const f32x4 bk = ld4(w.nr + off_b[k] + hh * 256 + 4 * lane);
          w.b[k][hh] = u32x2{pack_bf16x2(bk[0], bk[1]), pack_bf16x2(bk[2], bk[3])};
        }
      }
    }
    if constexpr (kX0) {
      w.tok = 0; w.at = 0.f; w.inv = 0.f;
      w.bw[0] = w.bw[1] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (lane < nrows) {
        const int64_t t = mb.token(row_base + lane);
        w.tok = (t < 0 || t >= Vp) ? 0 : (int)t;
        w.inv = x0_inv[row_base + lane];
        if (w.nr) w.at = w.nr[off_wte + w.tok];  // times the sign in ready()
      }
      if (w.nr) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) w.bw[hh] = ld4(w.nr + off_wte + Vp + hh * 256 + 4 * lane);
      }
    }
    w.lr = 1.f; w.l0 = 0.f;
    if (kMix || kXBase) {
      w.lr = resid_lambdas[layer];
      w.l0 = x0_lambdas[layer];
      if (w.nr) { w.lr = fmaf(w.s, w.nr[off_resid + layer], w.lr); w.l0 = fmaf(w.s, w.nr[off_x0 + layer], w.l0); }
    }
  }
  __device__ __forceinline__ void ready(Wave& w) const {
    w.d = ((w.dp[0] + w.dp[1]) + (w.dp[2] + w.dp[3])) + ((w.dp[4] + w.dp[5]) + (w.dp[6] + w.dp[7]));
    if constexpr (kX0) w.at *= w.s;
  }
  __device__ __forceinline__ void load(int row0, int, int lane, const Wave& w, Pre& p) const {
#pragma unroll
    for (int q = 0; q < kRows; ++q) {
      const int tq = kX0 ? lane_val(w.tok, row0 - w.row_base + q) : 0;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        if (!kXBase) p.xv[q][hh] = ld4(x + (int64_t)(row0 + q) * kD + hh * 256 + 4 * lane);
        if (kX0) p.x0v[q][hh] = ld4(wte + (int64_t)tq * kD + hh * 256 + 4 * lane);  // the embedding row
        else if (kMix) p.x0v[q][hh] = ld4(x0 + (int64_t)(row0 + q) * kD + hh * 256 + 4 * lane);
      }
    }
  }
  template <int R>
  __device__ __forceinline__ void rows(int row0, int, int, int lane, const Wave& w, const Pre& p,
                                       f32x4 (&v)[R][2]) const {
    static_assert(R == 4, "warp_sum4 reduces 4 rows");
    const int i0 = row0 - w.row_base;
    if constexpr (kJit) {
#pragma unroll
      for (int q = 0; q < R; ++q)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) v[q][hh] += jit.quad(mb, row0 + q, kD, hh * 256 + 4 * lane);
    }
    float ss[R];
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const float d = lane_val(w.d, i0 + q);
      const float at = kX0 ? lane_val(w.at, i0 + q) : 0.f, inv = kX0 ? lane_val(w.inv, i0 + q) : 0.f;
      ss[q] = 0.f;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        f32x4 xn = kXBase ? f32x4{0.f, 0.f, 0.f, 0.f} : p.xv[q][hh];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float val = v[q][hh][e];
          val += w.s * d * w.a[hh][e];
          const float x0e = kX0 ? fmaf(at, w.bw[hh][e], p.x0v[q][hh][e]) * inv : p.x0v[q][hh][e];
          if (kXBase) xn[e] = lambda_mix(w.lr, w.l0, x0e, x0e);  // block 0's input, as embed_kernel forms it
          xn[e] += val;
          if (kMix) xn[e] = lambda_mix(w.lr, w.l0, xn[e], x0e);
          ss[q] += xn[e] * xn[e];
        }
        v[q][hh] = xn;
        if (!kFinal) __builtin_nontemporal_store(xn, (f32x4*)(x + (int64_t)(row0 + q) * kD + hh * 256 + 4 * lane));
      }
    }
    const float tot = warp_sum4(ss, lane);
    float dk[kNDot][R];
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const float inv = rsq_norm(lane_val(tot, 16 * q) * (1.0f / kD) + kNormEps);
#pragma unroll
      for (int k = 0; k < kNDot; ++k) dk[k][q] = 0.f;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const uint32_t p0 = pack_bf16x2(v[q][hh][0] * inv, v[q][hh][1] * inv);
        const uint32_t p1 = pack_bf16x2(v[q][hh][2] * inv, v[q][hh][3] * inv);
        __builtin_nontemporal_store((u32x2{p0, p1}), (u32x2*)(h + (int64_t)(row0 + q) * kD + hh * 256 + 4 * lane));
#pragma unroll
        for (int k = 0; k < kNDot; ++k)
          dk[k][q] = dot2_bf16(p1, w.b[k][hh][1], dot2_bf16(p0, w.b[k][hh][0], dk[k][q]));
      }
    }
    if (w.nr) {
#pragma unroll
      for (int k = 0; k < kNDot; ++k) {
        const float dt = warp_sum4(dk[k], lane);
        if ((lane & 15) == 0) xb[(int64_t)(row0 + (lane >> 4)) * 4 + k] = dt;
      }
    }
  }
};

// hidden = relu(acc + s (x . b) a)^2 in bf16 (utils/model.py:107), and the next linear's rank-1 partial dot
// hidden . b_next over this 256-column tile (xb_next[row, n_tile]).
template <bool kJit>
struct EpiReluSqT {
  Members mb;
  bf16_t* out;
  int64_t ldo;
  int64_t off;
  const float* xb;  // [M, xb_ld]: column 0 holds x . b
  int xb_ld;
  int64_t off_next_b;   // noise offset of the next linear's b (its input is this output)
  float* xb_next;       // [M, n_tiles]
  int n_tiles;
  Jitter jit;           // kJit: the direct draws' jitter of the pre-activation
  static constexpr int kRows = kEpiRows;
  struct Wave {
    int row_base;
    const float* nr;
    float s, xb;
    f32x4 a;
    u32x2 b;  // the next linear's b at this lane's columns, as bf16 pairs (the reference's x @ b.to(bf16))
  };
  struct Pre {};
  __device__ __forceinline__ void begin(int row_base, int n0, int lane, int nrows, Wave& w) const {
    const int m = mb.member(row_base);
    w.row_base = row_base;
    w.nr = mb.nrow(m);
    w.s = 0.f; w.xb = 0.f;
    w.a = f32x4{0.f, 0.f, 0.f, 0.f};
    w.b = u32x2{0u, 0u};
    if (w.nr) {
      w.s = mb.sgn(m);
      w.a = ld4(w.nr + off + n0 + 4 * lane);
      const f32x4 bn = ld4(w.nr + off_next_b + n0 + 4 * lane);
      w.b = u32x2{pack_bf16x2(bn[0], bn[1]), pack_bf16x2(bn[2], bn[3])};
      if (lane < nrows) w.xb = xb[(int64_t)(row_base + lane) * xb_ld];
    }
  }
  __device__ __forceinline__ void load(int, int, int, const Wave&, Pre&) const {}
  template <int R>
  __device__ __forceinline__ void rows(int row0, int n0, int n_tile, int lane, const Wave& w, const Pre&,
                                       f32x4 (&v)[R]) const {
    if constexpr (kJit) {
#pragma unroll
      for (int q = 0; q < R; ++q) v[q] += jit.quad(mb, row0 + q, kF, n0 + 4 * lane);
    }
    if (w.nr) {
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const float k = lane_val(w.xb, row0 - w.row_base + q);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[q][e] += w.s * k * w.a[e];
      }
    }
    u32x2 pk[R];  // the bf16 outputs, which the next linear's rank-1 dots read back
#pragma unroll
    for (int q = 0; q < R; ++q) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float r = fmaxf(v[q][e], 0.f);
        v[q][e] = r * r;
      }
      pk[q] = u32x2{pack_bf16x2(v[q][0], v[q][1]), pack_bf16x2(v[q][2], v[q][3])};
      __builtin_nontemporal_store(pk[q], (u32x2*)(out + (int64_t)(row0 + q) * ldo + n0 + 4 * lane));
    }
    if (w.nr) {
      static_assert(R == 8, "warp_sum8 reduces 8 rows");
      float d[R];
#pragma unroll
      for (int q = 0; q < R; ++q) d[q] = dot2_bf16(pk[q][1], w.b[1], dot2_bf16(pk[q][0], w.b[0], 0.f));
      const float tot = warp_sum8(d, lane);
      if ((lane & 7) == 0) xb_next[(int64_t)(row0 + (lane >> 3)) * n_tiles + n_tile] = tot;
    }
  }
};
using EpiReluSq = EpiReluSqT<false>;

// logits z = 15 tanh((acc + s (h . b) a) / 15) (utils/model.py:203-204) and, per row of this 256-column tile, the sum
// over columns < vocab of exp(z - 15), plus the target's logit (utils/model.py:206-209). The soft cap keeps |z| < 15,
// so exp(z - 15) lies in (e^-30, 1]: the log-sum-exp needs no running maximum, lse = 15 + log(sum of the tile sums).
struct EpiHeadCE {
  Members mb;
  int64_t off;
  const float* xb;    // [M, xb_ld]: column 0 holds h . b
  int xb_ld;
  int vocab, n_part;
  float* part_sum;    // [M, n_part]
  float* tgt_logit;   // [M]
  const int64_t* targets;  // [n_seq, T]
  float* logits;      // [M, vocab] or NULL
  static constexpr int kRows = kEpiRows;
  // Columns in two halves over the XCD halves: each XCD keeps 2 MB of a 4 MB lm_head in its 4 MB L2 while the h rows
  // stream past (2.2 GB fetched per C4 launch against 5.4 GB in groups of 8 row panels, 1.15 GB compulsory).
  static constexpr int kNSplit = 2;
  struct Wave {
    int row_base, tg;  // tg: the lane's row's target, -1 when it is no column index (set in ready())
    int64_t t;         // the target as loaded
    const float* nr;
    float s, xb;
    f32x4 a;
  };
  struct Pre {};
  __device__ __forceinline__ void begin(int row_base, int n0, int lane, int nrows, Wave& w) const {
    const int m = mb.member(row_base);
    w.row_base = row_base;
    w.t = lane < nrows ? targets[(int64_t)mb.sq(m) * mb.T + (row_base - m * mb.T) + lane] : -1;
    w.tg = -1;
    w.nr = mb.nrow(m);
    w.s = 0.f; w.xb = 0.f;
    w.a = f32x4{0.f, 0.f, 0.f, 0.f};
    if (w.nr) {
      w.s = mb.sgn(m);
      w.a = ld4(w.nr + off + n0 + 4 * lane);
      if (lane < nrows) w.xb = xb[(int64_t)(row_base + lane) * xb_ld];
    }
  }
  __device__ __forceinline__ void ready(Wave& w) const { w.tg = (w.t >= 0 && w.t < vocab) ? (int)w.t : -1; }
  __device__ __forceinline__ void load(int, int, int, const Wave&, Pre&) const {}
  template <int R>
  __device__ __forceinline__ void rows(int row0, int n0, int n_tile, int lane, const Wave& w, const Pre&,
                                       f32x4 (&v)[R]) const {
    const int c0 = n0 + 4 * lane;
    const int i0 = row0 - w.row_base;
    if (w.nr) {
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const float k = lane_val(w.xb, i0 + q);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[q][e] += w.s * k * w.a[e];
      }
    }
    static_assert(R == 8, "warp_sum8 reduces 8 rows");
    // 15 tanh(u / 15) = 15 - 30 r with r = 1 / (exp(2 u / 15) + 1), so exp(z - 15) = exp2(g) with
    // g = -30 log2(e) r = 1 / ((exp(2 u / 15) + 1) / (-30 log2(e))): one fma and one rcp; z = 15 + g ln(2)
    constexpr float kCapIn = 2.0f / 15.0f * kLog2e, kCapInv = 1.0f / (-30.0f * kLog2e), kLn2 = 0.6931471805599453f;
    float se[R];
    if (n0 + 256 <= vocab && !logits) {
      // every column of the tile is a vocabulary column and no logits are written: no per-column branches; the
      // target's capped logit is recomputed by the one lane that holds it, with the operations of the path below
#pragma unroll
      for (int q = 0; q < R; ++q) {
        se[q] = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          se[q] += fast_exp2(fast_rcp(fmaf(fast_exp2(v[q][e] * kCapIn), kCapInv, kCapInv)));
        const int ti = lane_val(w.tg, i0 + q) - c0;
        if ((unsigned)ti < 4u) {
          const float vt = ti == 0 ? v[q][0] : ti == 1 ? v[q][1] : ti == 2 ? v[q][2] : v[q][3];
          tgt_logit[row0 + q] = fmaf(fast_rcp(fmaf(fast_exp2(vt * kCapIn), kCapInv, kCapInv)), kLn2, 15.0f);
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int row = row0 + q;
        const int tg = lane_val(w.tg, i0 + q);
        se[q] = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float g = fast_rcp(fmaf(fast_exp2(v[q][e] * kCapIn), kCapInv, kCapInv));
          const float z = fmaf(g, kLn2, 15.0f);
          if (c0 + e < vocab) {
            se[q] += fast_exp2(g);
            if (tg == c0 + e) tgt_logit[row] = z;
            if (logits) logits[(int64_t)row * vocab + c0 + e] = z;
          }
        }
      }
    }
    const float tot = warp_sum8(se, lane);
    if ((lane & 7) == 0) part_sum[(int64_t)(row0 + (lane >> 3)) * n_part + n_tile] = tot;
  }
};

// per-row CE from the column-tile sums: lse = 15 + log(sum); a negative target contributes 0, an out-of-range one NaN,
// and every token of a member with an out-of-range table entry NaN.
__global__ void ce_finalize_kernel(Members mb, const float* __restrict__ part_sum, int n_part,
                                   const float* __restrict__ tgt_logit, const int64_t* __restrict__ targets, int vocab,
                                   float* __restrict__ row_ce, float* __restrict__ token_loss, int64_t M) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= M) return;
  float sum = 0.f;
  for (int p = 0; p < n_part; ++p) sum += part_sum[r * n_part + p];
  const int m = mb.member(r);
  const int64_t tg = targets[(int64_t)mb.sq(m) * mb.T + (r - (int64_t)m * mb.T)];
  float ce;
  if (mb.bad(m)) ce = __builtin_nanf("");
  else if (tg < 0) ce = 0.f;
  else if (tg >= vocab) ce = __builtin_nanf("");
  else ce = 15.0f + logf(sum) - tgt_logit[r];
  row_ce[r] = ce;
  if (token_loss) token_loss[r] = ce;
}

// loss_sum[m] = sum over the member's T rows, a fixed-order tree (deterministic).
__global__ __launch_bounds__(256) void member_sum_kernel(const float* __restrict__ row_ce, int T, float* __restrict__ out) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  float s = 0.f;
  for (int t = threadIdx.x; t < T; t += 256) s += row_ce[(int64_t)m * T + t];
  s = warp_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[m] = (red[0] + red[1]) + (red[2] + red[3]);
}

using Tile = GemmShape<128, 256, 32, 2, 2, 3, 2>;  // two workgroups per CU: one's epilogue beside the other's MFMAs
// c_fc on 256 x 256 tiles of 8 waves (64 x 128 each, one workgroup per CU): its relu^2 epilogue is light, and the larger
// tile halves the weight re-reads per row (2.77 against 2.84 ms per C4 launch, alternating builds on one box; q|k|v
// and the head ran 2% and 14% slower on it). The one-workgroup-per-CU tiles take 64-deep K steps in two LDS stages:
// mlp_proj 2.73 against 2.98 ms per C4 launch and c_fc 2.69 against 2.72 (alternating builds, one box).
using FcTile = GemmShape<256, 256, 64, 4, 2, 2, 1>;
// Whole 512-wide rows, for the epilogues that normalize (both projections). attn_proj (K = 512) ran on 64 x 512 tiles
// at two workgroups per CU with 32-deep steps before: 1.41 ms per C4 launch against 1.34 on this tile.
using RowTile = GemmShape<128, 512, 64, 2, 4, 2>;
constexpr int kAttnOG = 1;  // 32 outputs per wave (4 waves per SIMD)

static inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

struct Workspace {
  float *x, *x0;
  bf16_t *h, *qkv, *y, *hid;
  float *xb, *gate, *xbp, *xb1, *psum, *tgt, *row_ce;
  u32x4* rope;  // [T, 16] per-lane rotary values of the q|k|v epilogue
  float* x0_inv;  // [M] embed_kernel's per-row norm scale (the mlp_proj epilogue recomputes x0 from it)
  size_t bytes;
};

static constexpr int kHeadParts = 4096 / Tile::BN;  // column tiles of the head GEMM at padded_vocab <= 4096

static Workspace carve(void* base, int64_t M, int64_t T) {
  Workspace w;
  char* p = (char*)base;
  size_t off = 0;
  auto take = [&](size_t n) { char* q = p + off; off += align256(n); return (void*)q; };
  w.x = (float*)take(M * kD * 4);
  w.x0 = (float*)take(M * kD * 4);
  w.h = (bf16_t*)take(M * kD * 2);
  w.qkv = (bf16_t*)take(M * kQKV * 2);
  w.y = (bf16_t*)take(M * kD * 2);
  w.hid = (bf16_t*)take(M * kF * 2);
  w.xb = (float*)take(M * 4 * 4);
  w.gate = (float*)take(M * kH * 4);
  w.xbp = (float*)take(M * kH * 4);
  w.xb1 = (float*)take(M * (kF / Tile::BN) * 4);
  w.psum = (float*)take(M * kHeadParts * 4);
  w.tgt = (float*)take(M * 4);
  w.row_ce = (float*)take(M * 4);
  w.x0_inv = (float*)take(M * 4);
  w.rope = (u32x4*)take(T * 16 * sizeof(u32x4));
  w.bytes = off;
  return w;
}

// The q|k|v epilogue's rotary values, per position t and lane l of a head's 16 (channels 4l .. 4l+3): cos of
// frequency pair 4 (l % 8) + e as bf16 pairs, then sin with the rotation's sign, + on the first half (channels < 32)
// and - on the second (utils/model.py:55-58). The model's tables hold bf16 values, so the packing is exact.
__global__ __launch_bounds__(256) void rope_table_kernel(const float* __restrict__ cos_t,
                                                         const float* __restrict__ sin_t, int64_t T,
                                                         u32x4* __restrict__ rope) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // t * 16 + l
  if (i >= T * 16) return;
  const int64_t t = i >> 4;
  const int l = (int)(i & 15), j = 4 * (l & 7);
  const f32x4 c = *(const f32x4*)(cos_t + t * 32 + j);
  f32x4 sn = *(const f32x4*)(sin_t + t * 32 + j);
  if (l >= 8) sn = -sn;
  rope[i] = u32x4{pack_bf16x2(c[0], c[1]), pack_bf16x2(c[2], c[3]), pack_bf16x2(sn[0], sn[1]), pack_bf16x2(sn[2], sn[3])};
}

// dst[r] = norm(src[r]) in fp32, one wave per row (the MLP's input as the capture keeps it)
__global__ __launch_bounds__(256) void rms_rows_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                       int64_t M) {
  const int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= M) return;
  const int c0 = (threadIdx.x & 63) * 8;
  const f32x4 v0 = *(const f32x4*)(src + r * kD + c0), v1 = *(const f32x4*)(src + r * kD + c0 + 4);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) ss += v0[j] * v0[j] + v1[j] * v1[j];
  const float inv = rsq_norm(warp_sum(ss) * (1.0f / kD) + kNormEps);
  *(f32x4*)(dst + r * kD + c0) = f32x4{v0[0] * inv, v0[1] * inv, v0[2] * inv, v0[3] * inv};
  *(f32x4*)(dst + r * kD + c0 + 4) = f32x4{v1[0] * inv, v1[1] * inv, v1[2] * inv, v1[3] * inv};
}

// dst[r] = src[the member's batch row, same position]: the captured block input replicated over the draws
__global__ __launch_bounds__(256) void replicate_rows_kernel(Members mb, const float* __restrict__ src,
                                                             float* __restrict__ dst, int64_t M) {
  const int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= M) return;
  const int lane = threadIdx.x & 63, m = mb.member(r);
  const float* s = src + ((int64_t)mb.sq(m) * mb.T + (r - (int64_t)m * mb.T)) * kD + lane * 8;
  float* d = dst + r * kD + lane * 8;
  *(f32x4*)d = *(const f32x4*)s;
  *(f32x4*)(d + 4) = *(const f32x4*)(s + 4);
}

// member m of the direct draws: batch row m % n_seq (members are draw-major)
__global__ void member_rows_kernel(int32_t* __restrict__ seq, int64_t members, int64_t n_seq) {
  const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (m < members) seq[m] = (int32_t)(m % n_seq);
}

static bool g_prepared = false;
static int prepare_all() {
  if (g_prepared) return NOISE_OK;
  NOISE_CHECK_HIP((prepare_gemm<Tile, EpiQKV>()));
  NOISE_CHECK_HIP((prepare_gemm<RowTile, EpiResidNorm<false, 1, false, false, true>>()));
  NOISE_CHECK_HIP((prepare_gemm<RowTile, EpiResidNorm<true, 3>>()));
  NOISE_CHECK_HIP((prepare_gemm<FcTile, EpiReluSq>()));
  NOISE_CHECK_HIP((prepare_gemm<FcTile, EpiReluSqT<true>>()));
  NOISE_CHECK_HIP((prepare_gemm<RowTile, EpiResidNorm<false, 1, true, false, true>>()));
  NOISE_CHECK_HIP((prepare_gemm<RowTile, EpiResidNorm<true, 3, true>>()));
  NOISE_CHECK_HIP((prepare_gemm<RowTile, EpiResidNorm<true, 3, false, true>>()));
  NOISE_CHECK_HIP((prepare_gemm<RowTile, EpiResidNorm<false, 1>>()));
  NOISE_CHECK_HIP((prepare_gemm<RowTile, EpiResidNorm<false, 1, true>>()));
  NOISE_CHECK_HIP((prepare_gemm<RowTile, EpiResidNorm<false, 1, false, true, false, true>>()));
  NOISE_CHECK_HIP((prepare_gemm<Tile, EpiHeadCE>()));
  g_prepared = true;
  return NOISE_OK;
}

}  // namespace noise

using namespace noise;

extern "C" size_t noise_population_forward_workspace(int64_t members, int64_t T) {
  if (members <= 0 || T <= 0) return 0;
  return carve(nullptr, members * T, T).bytes;
}

// The direct draws' part of a forward (train/val/dust.py:195-233): a clean pass that captures every block's input
// (capture != NULL), or a rerun of blocks entry .. n_layer - 1 from a captured input with jitter at sites of block
// `entry` (entry -1: the token embedding's jitter, every block rerun).
struct DustRun {
  int entry;
  const float* x_in;
  const float* x0_in;
  int sites;  // bit s: jitter site s (0 embedding, 1 attention output, 2 attn.c_proj, 3 mlp.c_fc, 4 mlp.c_proj)
  float sigma;
  uint64_t seed;
  int draw0, n_seq;
  float* capture;  // [n_layer + 1, M, 512]: block inputs, then x0
  // optional, [n_layer, M, width] bf16: the inputs of the writers' linears, for reassembling weight errors
  bf16_t* cap_attn;  // attn.c_proj's input (the attention output), width 512
  float* cap_fc;     // mlp.c_fc's input (the MLP's normed input, fp32 as the reference's F.rms_norm gives it), 512
  bf16_t* cap_mlp;   // mlp.c_proj's input (relu² of c_fc), width 2048
  // the jitter of site s when it is set and block i is the entry
  Jitter jit(int i, int s) const {
    Jitter j;
    memset(&j, 0, sizeof(j));
    if (((sites >> s) & 1) && (s == 0 ? entry < 0 : i == entry)) {
      j.sigma = sigma; j.site = (uint32_t)s; j.seed = seed; j.draw0 = draw0; j.n_seq = n_seq;
    }
    return j;
  }
};

static int forward_impl(const noise_gpt* model, const noise_perturbation* pert, const int64_t* tokens,
                        const int64_t* targets, int64_t n_seq, int64_t T, const int32_t* member_seq,
                        const int32_t* member_row, const float* member_sign, int64_t members, float* loss_sum,
                        float* token_loss, float* logits, void* workspace, size_t workspace_bytes, hipStream_t stream,
                        const DustRun* dr) {
  NOISE_REQUIRE(model && pert, "model / perturbation is NULL");
  NOISE_REQUIRE(members > 0 && n_seq > 0, "members and n_seq must be positive");
  NOISE_REQUIRE(members <= 65535, "members = %lld: at most 65535 per call (the attention grid's z dimension)",
                (long long)members);
  NOISE_REQUIRE(T > 0 && T % 128 == 0, "T = %lld must be a positive multiple of 128", (long long)T);
  NOISE_REQUIRE(model->n_layer > 0 && model->n_layer <= NOISE_MAX_LAYERS, "n_layer %d outside [1, %d]", model->n_layer,
                NOISE_MAX_LAYERS);
  NOISE_REQUIRE(model->padded_vocab > 0 && model->padded_vocab % Tile::BN == 0 && model->padded_vocab <= 4096,
                "padded_vocab %d must be a multiple of %d and <= 4096", model->padded_vocab, Tile::BN);
  NOISE_REQUIRE(model->vocab > 0 && model->vocab <= model->padded_vocab, "vocab %d outside [1, padded_vocab]",
                model->vocab);
  NOISE_REQUIRE(tokens && member_seq && member_row && member_sign, "tokens / member tables are NULL");
  NOISE_REQUIRE(targets || logits, "need targets (losses) or logits");
  NOISE_REQUIRE(model->wte && model->lm_head && model->rope_cos && model->rope_sin && model->resid_lambdas &&
                    model->x0_lambdas, "model weight pointer is NULL");
  const int64_t M = members * T;
  NOISE_REQUIRE(M <= (int64_t)INT32_MAX / 4, "members * T = %lld too large", (long long)M);
  Workspace ws = carve(workspace, M, T);
  NOISE_REQUIRE(workspace && workspace_bytes >= ws.bytes, "workspace %zu bytes < %zu", workspace_bytes, ws.bytes);
  int rc = prepare_all();
  if (rc) return rc;

  NOISE_REQUIRE(!pert->rows || (pert->n_rows > 0 && pert->n_rows <= INT32_MAX && pert->stride > 0),
                "perturbation rows given: n_rows = %lld must be in [1, 2^31) and the stride positive",
                (long long)pert->n_rows);
  // member tables are read on the device: an entry outside [0, n_seq) or [0, n_rows) makes that member's loss NaN
  Members mb{(int)T, member_seq, member_row, member_sign, pert->rows, pert->stride, tokens, n_seq, pert->n_rows};
  const int Vp = model->padded_vocab;
  const bool noisy = pert->rows != nullptr;
  const unsigned row_blocks = (unsigned)((M + 3) / 4);
  DustRun none;
  memset(&none, 0, sizeof(none));
  none.entry = -1;
  if (!dr) dr = &none;
  const bool from_block = dr->entry >= 0;  // rerun from a captured block input
  const int first_layer = from_block ? dr->entry : 0;
  // the λ mix recomputes x0 from the embedding table when this call's embed_kernel formed it without jitter
  const bool x0_recompute = !from_block && !dr->jit(-1, 0).on();
  // and block 0's attn c_proj rebuilds block 0's input from x0 too, so the embedding kernel stores no x (a capture
  // keeps the stored x: it copies every block's input)
  const bool x_from_x0 = x0_recompute && !dr->capture;

  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((T * 16 + 255) / 256)), dim3(256), 0, stream, model->rope_cos,
                     model->rope_sin, T, ws.rope);
  NOISE_LAUNCH_CHECK();
  if (from_block) {
    hipLaunchKernelGGL(replicate_rows_kernel, dim3(row_blocks), dim3(256), 0, stream, mb, dr->x_in, ws.x, M);
    NOISE_LAUNCH_CHECK();
    hipLaunchKernelGGL(replicate_rows_kernel, dim3(row_blocks), dim3(256), 0, stream, mb, dr->x0_in, ws.x0, M);
    NOISE_LAUNCH_CHECK();
  } else {
    NoiseTimer tm(kTimeEmbed, stream);
    EmbedMix em;
    memset(&em, 0, sizeof(em));
    em.x = ws.x; em.h = ws.h; em.xb = ws.xb;
    em.resid_lambdas = model->resid_lambdas; em.x0_lambdas = model->x0_lambdas;
    em.off_resid = pert->resid_lambdas; em.off_x0 = pert->x0_lambdas;
    em.off_b[0] = pert->c_q[0] + kD; em.off_b[1] = pert->c_k[0] + kD; em.off_b[2] = pert->c_v[0] + kD;
    em.write_x0 = dr->capture != nullptr || !x0_recompute;
    em.write_x = !x_from_x0;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((M + 31) / 32)), dim3(256), 0, stream, mb, model->wte, Vp, pert->wte,
                       dr->jit(-1, 0), ws.x0, ws.x0_inv, em, M);
    NOISE_LAUNCH_CHECK();
  }
  if (dr->capture)
    NOISE_CHECK_HIP(hipMemcpyAsync(dr->capture + (int64_t)model->n_layer * M * kD, ws.x0, (size_t)M * kD * 4,
                                   hipMemcpyDeviceToDevice, stream));

  for (int i = first_layer; i < model->n_layer; ++i) {
    const noise_layer& L = model->layers[i];
    NOISE_REQUIRE(L.w_qkv && L.w_proj && L.w_fc && L.w_mlp_proj, "layer %d weight pointer is NULL", i);
    NOISE_REQUIRE((L.w_gate == nullptr) == (L.ve == nullptr), "layer %d: w_gate and ve must both be set or both NULL", i);
    NOISE_REQUIRE(L.window >= 0, "layer %d: negative window", i);
    if (i == first_layer && from_block) {
      // a rerun from a captured block input starts from the mixed x: norm, q/k/v dots and gate (block 0's come from
      // the embedding kernel, later blocks' from the epilogue of the previous block's MLP projection)
      NormArgs na;
      memset(&na, 0, sizeof(na));
      na.x = ws.x; na.x0 = ws.x0; na.mix = 0; na.first = 0;
      na.resid_lambdas = model->resid_lambdas; na.x0_lambdas = model->x0_lambdas; na.layer = 0;
      na.off_resid = pert->resid_lambdas; na.off_x0 = pert->x0_lambdas;
      na.h = ws.h; na.ndot = 3;
      na.off_b[0] = pert->c_q[0] + kD; na.off_b[1] = pert->c_k[0] + kD; na.off_b[2] = pert->c_v[0] + kD;
      na.xb = ws.xb; na.w_gate = L.w_gate; na.off_gate = pert->ve_gate[0]; na.gate = ws.gate; na.M = M;
      NoiseTimer tm(kTimeNorm, stream);
      hipLaunchKernelGGL(mix_norm_kernel, dim3(row_blocks), dim3(256), 0, stream, mb, na);
      NOISE_LAUNCH_CHECK();
    } else if (L.w_gate) {  // the value-embedding gate from h
      NoiseTimer tm(kTimeNorm, stream);
      hipLaunchKernelGGL(gate_kernel, dim3((unsigned)((M + 31) / 32)), dim3(256), 0, stream, mb, ws.h, L.w_gate,
                         pert->ve_gate[i], ws.gate, M);
      NOISE_LAUNCH_CHECK();
    }
    if (dr->capture)  // x now holds block i's (mixed) input
      NOISE_CHECK_HIP(hipMemcpyAsync(dr->capture + (int64_t)i * M * kD, ws.x, (size_t)M * kD * 4,
                                     hipMemcpyDeviceToDevice, stream));

    EpiQKV eq{mb, ws.qkv, {pert->c_q[i], pert->c_k[i], pert->c_v[i]}, ws.xb, L.w_gate ? ws.gate : nullptr, L.ve,
              pert->ve[i], Vp, ws.rope};
    {
      NoiseTimer tm(kTimeQKV, stream);
      NOISE_CHECK_HIP((launch_gemm<Tile>(ws.h, kD, L.w_qkv, kD, (int)M, kQKV, kD, eq, stream)));
    }

    FlashArgs fa;
    memset(&fa, 0, sizeof(fa));
    fa.x = ws.qkv; fa.y = ws.qkv + kD; fa.v = ws.qkv + 2 * kD;
    fa.x_sb = fa.y_sb = fa.v_sb = T * kQKV; fa.x_st = fa.y_st = fa.v_st = kQKV;
    fa.out = ws.y; fa.o_sb = T * kD; fa.o_st = kD;
    fa.xb_out = noisy ? ws.xbp : nullptr;
    fa.xb_vec = noisy ? pert->rows + pert->c_proj[i] + kD : nullptr;
    fa.xb_row = member_row; fa.xb_stride = pert->stride; fa.xb_rows = pert->n_rows;
    fa.heads = kH; fa.T = (int)T; fa.window = L.window;
    {
      const Jitter jo = dr->jit(i, 1);
      fa.jit_sigma = jo.sigma; fa.jit_site = jo.site; fa.jit_seed = jo.seed; fa.jit_draw0 = jo.draw0;
      fa.jit_n_seq = jo.n_seq > 0 ? jo.n_seq : 1; fa.jit_seq = member_seq;
    }
    {
      NoiseTimer tm(kTimeAttention, stream);
      // the bounded softmax: q and k are RMS-normed over 64 channels, so |q . k| / 8 <= 8
      NOISE_CHECK_HIP((launch_flash<kAttn, true, kAttnOG>(fa, members, kH, stream)));
    }
    if (dr->cap_attn)
      NOISE_CHECK_HIP(hipMemcpyAsync(dr->cap_attn + (int64_t)i * M * kD, ws.y, (size_t)M * kD * 2,
                                     hipMemcpyDeviceToDevice, stream));

    // attention projection + residual, then the MLP's norm and c_fc's rank-1 dot
    EpiResidNorm<false, 1> ep;
    memset(&ep, 0, sizeof(ep));
    ep.mb = mb; ep.x = ws.x; ep.xbp = ws.xbp; ep.nxb = kH; ep.off = pert->c_proj[i];
    ep.h = ws.h; ep.off_b[0] = pert->c_fc[i] + kF;  // c_fc's a spans its 2048 outputs
    ep.xb = ws.xb;
    {
      NoiseTimer tm(kTimeProj, stream);
      const Jitter jp = dr->jit(i, 2);
      if (jp.on()) {
        EpiResidNorm<false, 1, true> ej;
        memcpy((void*)&ej, (const void*)&ep, sizeof(ep));
        ej.jit = jp;
        NOISE_CHECK_HIP((launch_gemm<RowTile>(ws.y, kD, L.w_proj, kD, (int)M, kD, kD, ej, stream)));
      } else if (i == 0 && x_from_x0) {
        EpiResidNorm<false, 1, false, true, false, true> eb;
        memcpy((void*)&eb, (const void*)&ep, sizeof(ep));
        eb.wte = model->wte; eb.x0_inv = ws.x0_inv; eb.Vp = Vp; eb.off_wte = pert->wte;
        eb.resid_lambdas = model->resid_lambdas; eb.x0_lambdas = model->x0_lambdas; eb.layer = 0;
        eb.off_resid = pert->resid_lambdas; eb.off_x0 = pert->x0_lambdas;
        NOISE_CHECK_HIP((launch_gemm<RowTile>(ws.y, kD, L.w_proj, kD, (int)M, kD, kD, eb, stream)));
      } else {
        NOISE_CHECK_HIP((launch_gemm<RowTile>(ws.y, kD, L.w_proj, kD, (int)M, kD, kD, ep, stream)));
      }
    }

    if (dr->cap_fc) {
      hipLaunchKernelGGL(rms_rows_kernel, dim3(row_blocks), dim3(256), 0, stream, ws.x, dr->cap_fc + (int64_t)i * M * kD,
                         M);
      NOISE_LAUNCH_CHECK();
    }
    {
      NoiseTimer tm(kTimeFc, stream);
      const Jitter jf = dr->jit(i, 3);
      if (jf.on()) {
        EpiReluSqT<true> er{mb, ws.hid, kF, pert->c_fc[i], ws.xb, 4, pert->mlp_proj[i] + kD, ws.xb1, kF / Tile::BN, jf};
        NOISE_CHECK_HIP((launch_gemm<FcTile>(ws.h, kD, L.w_fc, kD, (int)M, kF, kD, er, stream)));
      } else {
        EpiReluSq er{mb, ws.hid, kF, pert->c_fc[i], ws.xb, 4, pert->mlp_proj[i] + kD, ws.xb1, kF / Tile::BN, Jitter{}};
        NOISE_CHECK_HIP((launch_gemm<FcTile>(ws.h, kD, L.w_fc, kD, (int)M, kF, kD, er, stream)));
      }
    }

    if (dr->cap_mlp)
      NOISE_CHECK_HIP(hipMemcpyAsync(dr->cap_mlp + (int64_t)i * M * kF, ws.hid, (size_t)M * kF * 2,
                                     hipMemcpyDeviceToDevice, stream));

    // MLP projection + residual, then the next block's lambda mix, norm and q/k/v dots (or the final norm and
    // lm_head's rank-1 dot)
    const bool last = i + 1 == model->n_layer;
    if (last) {
      EpiResidNorm<false, 1, false, false, true> em;  // after the last block only h and the head's dot are read
      memset(&em, 0, sizeof(em));
      em.mb = mb; em.x = ws.x; em.xbp = ws.xb1; em.nxb = kF / Tile::BN; em.off = pert->mlp_proj[i];
      em.h = ws.h; em.xb = ws.xb; em.off_b[0] = pert->lm_head + Vp;
      NoiseTimer tm(kTimeMlpProj, stream);
      const Jitter jm = dr->jit(i, 4);
      if (jm.on()) {
        EpiResidNorm<false, 1, true, false, true> ej;
        memcpy((void*)&ej, (const void*)&em, sizeof(em));
        ej.jit = jm;
        NOISE_CHECK_HIP((launch_gemm<RowTile>(ws.hid, kF, L.w_mlp_proj, kF, (int)M, kD, kF, ej, stream)));
      } else {
        NOISE_CHECK_HIP((launch_gemm<RowTile>(ws.hid, kF, L.w_mlp_proj, kF, (int)M, kD, kF, em, stream)));
      }
    } else {
      EpiResidNorm<true, 3> em;
      memset(&em, 0, sizeof(em));
      em.mb = mb; em.x = ws.x; em.xbp = ws.xb1; em.nxb = kF / Tile::BN; em.off = pert->mlp_proj[i];
      em.h = ws.h; em.xb = ws.xb;
      em.x0 = ws.x0; em.resid_lambdas = model->resid_lambdas; em.x0_lambdas = model->x0_lambdas;
      em.layer = i + 1; em.off_resid = pert->resid_lambdas; em.off_x0 = pert->x0_lambdas;
      em.off_b[0] = pert->c_q[i + 1] + kD; em.off_b[1] = pert->c_k[i + 1] + kD; em.off_b[2] = pert->c_v[i + 1] + kD;
      NoiseTimer tm(kTimeMlpProj, stream);
      const Jitter jm = dr->jit(i, 4);
      if (jm.on()) {
        EpiResidNorm<true, 3, true> ej;
        memcpy((void*)&ej, (const void*)&em, sizeof(em));
        ej.jit = jm;
        NOISE_CHECK_HIP((launch_gemm<RowTile>(ws.hid, kF, L.w_mlp_proj, kF, (int)M, kD, kF, ej, stream)));
      } else if (x0_recompute) {
        EpiResidNorm<true, 3, false, true> ex;
        memcpy((void*)&ex, (const void*)&em, sizeof(em));
        ex.wte = model->wte; ex.x0_inv = ws.x0_inv; ex.Vp = Vp; ex.off_wte = pert->wte;
        NOISE_CHECK_HIP((launch_gemm<RowTile>(ws.hid, kF, L.w_mlp_proj, kF, (int)M, kD, kF, ex, stream)));
      } else {
        NOISE_CHECK_HIP((launch_gemm<RowTile>(ws.hid, kF, L.w_mlp_proj, kF, (int)M, kD, kF, em, stream)));
      }
    }
  }

  const int n_part = Vp / Tile::BN;
  const int64_t* tg = targets ? targets : tokens;  // logits-only calls still run the CE bookkeeping on tokens
  EpiHeadCE eh{mb, pert->lm_head, ws.xb, 4, model->vocab, n_part, ws.psum, ws.tgt, tg, logits};
  {
    NoiseTimer tm(kTimeHead, stream);
    NOISE_CHECK_HIP((launch_gemm<Tile>(ws.h, kD, model->lm_head, kD, (int)M, Vp, kD, eh, stream)));
  }
  if (targets && (loss_sum || token_loss)) {
    NoiseTimer tm(kTimeCeFinal, stream);
    hipLaunchKernelGGL(ce_finalize_kernel, dim3((unsigned)((M + 255) / 256)), dim3(256), 0, stream, mb, ws.psum, n_part,
                       ws.tgt, targets, model->vocab, ws.row_ce, token_loss, M);
    NOISE_LAUNCH_CHECK();
    if (loss_sum) {
      hipLaunchKernelGGL(member_sum_kernel, dim3((unsigned)members), dim3(256), 0, stream, ws.row_ce, (int)T, loss_sum);
      NOISE_LAUNCH_CHECK();
    }
  }
  return NOISE_OK;
}

extern "C" int noise_population_forward(const noise_gpt* model, const noise_perturbation* pert, const int64_t* tokens,
                                        const int64_t* targets, int64_t n_seq, int64_t T, const int32_t* member_seq,
                                        const int32_t* member_row, const float* member_sign, int64_t members,
                                        float* loss_sum, float* token_loss, float* logits, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return forward_impl(model, pert, tokens, targets, n_seq, T, member_seq, member_row, member_sign, members, loss_sum,
                      token_loss, logits, workspace, workspace_bytes, (hipStream_t)stream, nullptr);
}

// ---- the direct draws (train/val/dust.py:195-233) ------------------------------------------------------------

extern "C" size_t noise_dust_workspace(int64_t n_draws, int64_t n_seq, int64_t T) {
  if (n_draws <= 0 || n_seq <= 0 || T <= 0) return 0;
  const int64_t members = n_draws * n_seq;
  return align256((size_t)members * 4) + carve(nullptr, members * T, T).bytes;
}

// members = n_draws * n_seq (draw-major, member m on batch row m % n_seq), clean weights; per-token CE out
static int dust_forward(const noise_gpt* model, const int64_t* tokens, const int64_t* targets, int64_t n_seq, int64_t T,
                        int64_t n_draws, float* token_loss, void* workspace, size_t workspace_bytes, hipStream_t stream,
                        const DustRun& dr) {
  NOISE_REQUIRE(model && tokens && targets && token_loss, "NULL pointer argument");
  NOISE_REQUIRE(n_seq > 0 && n_draws > 0 && T > 0, "n_seq, n_draws and T must be positive");
  NOISE_REQUIRE((int64_t)n_draws * n_seq <= 65535, "n_draws * n_seq = %lld: at most 65535 per call",
                (long long)n_draws * n_seq);
  const int64_t members = n_draws * n_seq;
  NOISE_REQUIRE(workspace && workspace_bytes >= noise_dust_workspace(n_draws, n_seq, T), "workspace too small");
  int32_t* seq = (int32_t*)workspace;
  const size_t head = align256((size_t)members * 4);
  hipLaunchKernelGGL(member_rows_kernel, dim3((unsigned)((members + 255) / 256)), dim3(256), 0, stream, seq, members,
                     n_seq);
  NOISE_LAUNCH_CHECK();
  noise_perturbation clean;
  memset(&clean, 0, sizeof(clean));  // rows == NULL: no weight noise
  if (!dr.capture) {
    NoiseTimer tm(kTimeDustRerun, stream);
    return forward_impl(model, &clean, tokens, targets, n_seq, T, seq, seq, (const float*)seq, members, nullptr,
                        token_loss, nullptr, (char*)workspace + head, workspace_bytes - head, stream, &dr);
  }
  return forward_impl(model, &clean, tokens, targets, n_seq, T, seq, seq, (const float*)seq, members, nullptr,
                      token_loss, nullptr, (char*)workspace + head, workspace_bytes - head, stream, &dr);
}

extern "C" int noise_dust_capture_sites(const noise_gpt* model, const int64_t* tokens, const int64_t* targets,
                                        int64_t n_seq, int64_t T, float* token_loss, float* capture,
                                        uint16_t* attn_in, float* fc_in, uint16_t* mlp_in, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  NOISE_REQUIRE(capture, "capture is NULL");
  DustRun dr;
  memset(&dr, 0, sizeof(dr));
  dr.entry = -1; dr.n_seq = (int)n_seq; dr.capture = capture;
  dr.cap_attn = (bf16_t*)attn_in; dr.cap_fc = fc_in; dr.cap_mlp = (bf16_t*)mlp_in;
  return dust_forward(model, tokens, targets, n_seq, T, 1, token_loss, workspace, workspace_bytes,
                      (hipStream_t)stream, dr);
}

extern "C" int noise_dust_capture(const noise_gpt* model, const int64_t* tokens, const int64_t* targets, int64_t n_seq,
                                  int64_t T, float* token_loss, float* capture, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  return noise_dust_capture_sites(model, tokens, targets, n_seq, T, token_loss, capture, nullptr, nullptr, nullptr,
                                  workspace, workspace_bytes, stream);
}

extern "C" int noise_dust_rerun(const noise_gpt* model, const noise_dust_draws* d, const int64_t* tokens,
                                const int64_t* targets, int64_t n_seq, int64_t T, float* token_loss, void* workspace,
                                size_t workspace_bytes, void* stream) {
  NOISE_REQUIRE(model && d, "NULL pointer argument");
  NOISE_REQUIRE(d->entry >= -1 && d->entry < model->n_layer, "entry %d outside [-1, n_layer)", d->entry);
  NOISE_REQUIRE(d->n_draws > 0 && d->draw0 >= 0 && d->sigma >= 0.f, "n_draws > 0, draw0 >= 0, sigma >= 0 needed");
  NOISE_REQUIRE(d->entry < 0 ? (d->sites & ~1) == 0 : (d->sites & ~0x1E) == 0,
                "sites 0x%x do not belong to entry %d (embedding: bit 0; a block: bits 1-4)", d->sites, d->entry);
  NOISE_REQUIRE(d->entry < 0 || (d->x_in && d->x0_in), "a rerun from block %d needs its captured input and x0",
                d->entry);
  NOISE_REQUIRE(n_seq <= (int64_t)1 << 20 && (int64_t)d->n_draws * n_seq * T <= (int64_t)INT32_MAX / 4,
                "n_draws * n_seq * T too large");
  DustRun dr;
  memset(&dr, 0, sizeof(dr));
  dr.entry = d->entry; dr.x_in = d->x_in; dr.x0_in = d->x0_in; dr.sites = d->sites; dr.sigma = d->sigma;
  dr.seed = d->seed; dr.draw0 = d->draw0; dr.n_seq = (int)n_seq;
  return dust_forward(model, tokens, targets, n_seq, T, d->n_draws, token_loss, workspace, workspace_bytes,
                      (hipStream_t)stream, dr);
}
