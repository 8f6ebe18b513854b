/* noise_amd — C ABI of the MI355X (gfx950) kernels behind Noise's forward-only population training hot path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t (passed as void*), launches on that stream
 * without synchronizing, allocates nothing, and returns 0 or a NOISE_ERR_* code; noise_last_error() then holds a
 * message. Tensors are contiguous row-major unless a stride argument says otherwise. "bf16" buffers are uint16_t
 * bfloat16 bit patterns. Citations are relative to the reference checkout (qlabs-eng/noise).
 */
#ifndef NOISE_AMD_H
#define NOISE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NOISE_OK 0
#define NOISE_ERR_ARG 1   /* bad shape, size, pointer or configuration: Python raises ValueError */
#define NOISE_ERR_HIP 2   /* a HIP runtime call failed: Python raises RuntimeError */
#define NOISE_ERR_WORKSPACE 3 /* workspace too small: Python raises ValueError */

#define NOISE_MAX_LAYERS 16

/* Message of the last failed call on this thread. */
const char* noise_last_error(void);
/* ABI version (bumped on any signature change or added entry point). */
int noise_abi_version(void);

/* Launch timing for measurement (no counterpart in the reference, whose kernels are timed with CUDA events from
 * Python: train/speedrun/run.py:4262, 4316): noise_timing_enable(1) clears the figures and brackets every following
 * launch with hipEvents on its stream; noise_timing_read() waits for them and returns per-class launch counts and
 * summed milliseconds (arrays of n entries) and the class names; it returns the number of classes. */
int noise_timing_enable(int enable);
int noise_timing_read(int32_t n, int64_t* counts, double* total_ms, const char** names);

/* Measured ceiling for the roofline (no counterpart in the reference, which publishes no kernel rates): a sustained
 * stream of v_mfma_f32_32x32x16_bf16 over `workgroups` workgroups of 4 waves, each wave `iters` steps of 8 MFMAs
 * (32,768 FLOP each) on 8 independent accumulators. ops bf16 [n_frag_rows, 64 lanes, 8] (n_frag_rows >= 32) supplies
 * the operand bits (the engine clock under load depends on them); lds = 0 holds each wave's 6 fragments in registers,
 * lds = 1 reads every step's 6 fragments from a 32 KB LDS block (iters even), as a GEMM main loop does. out fp32
 * [workgroups * 256]. FLOPs = workgroups * 4 * iters * 8 * 32768. */
int noise_peak_mfma(const uint16_t* ops, int64_t n_frag_rows, int32_t iters, int32_t workgroups, int32_t lds,
                    float* out, void* stream);

/* ---- a1: counter-based noise (replaces the 2^28-value torch.randn buffer and the torch.randint offsets) -------- */

/* out[j] = G[start + j], the virtual N(0,1) buffer of Philox4x32-10 + Box-Muller values.
 * Replaces: archive/10M/train/val/eggroll.py:114 (torch.randn(NOISE, generator=manual_seed(SEED))). */
int noise_rng_buffer(uint64_t seed, uint64_t start, int64_t n, float* out, void* stream);

/* out[p * pairs + d] = offset of direction d of parameter p at this step, an integer in [0, 2^28 - widths[p]);
 * widths (host array [n_params], n_params <= 128: every model of up to NOISE_MAX_LAYERS blocks) = sum(shape) of each
 * parameter in named_parameters() order.
 * Replaces: archive/10M/train/val/eggroll.py:117-120 (Eggroll.offsets). */
int noise_rng_offsets(uint64_t seed, uint64_t step, const int64_t* widths, int32_t n_params, int64_t pairs,
                      int64_t* out, void* stream);

/* rows[j, col0[p] + e] = G[offsets[p * pairs + directions[j]] + e] for e < widths[p]: the noise of n directions,
 * every parameter's (a | b) slice side by side (col0 = prefix sums of widths, row stride = sum of widths); widths is
 * a host array of n_params <= 128 entries; a direction outside [0, pairs) yields a row of NaN.
 * Replaces: archive/10M/train/val/eggroll.py:122-128 (Eggroll.noise). */
int noise_rng_rows(uint64_t seed, const int64_t* offsets, int64_t pairs, const int64_t* widths, int32_t n_params,
                   const int64_t* directions, int64_t n, float* rows, void* stream);

/* ---- a2: perturbed linear --------------------------------------------------------------------------------- */

/* y[i, t, :] = c[t, :] + sign[i] u_i[t] a_i in fp32, with c = bf16(x W^T), u_i[t] = bf16(x[t] . bf16(b_i)) and a_i
 * rounded to bf16 (the reference's bf16 autocast arithmetic); a_i = noise[i * noise_stride + a_off + (0..out)],
 * b_i = noise[i * noise_stride + b_off + (0..in)]; W bf16 [out, in]. Outputs (either may be NULL): y fp32 [m, T, out];
 * sumsq fp32 [m] = sum of y_i^2 per member.
 *   x_shared = 0: x bf16 [m, T, in], one GEMM over the m T rows; T % 128 == 0.
 *   x_shared = 1: x bf16 [T, in] shared by every member (config 2): x W^T once per 256 x 256 tile, every
 *                 member's term from that tile. With y == NULL, sumsq by the expanded square (the per-member sums
 *                 sum_c a_i[c] sum_t u_i[t] c[t, c] on the MFMA units); with y, every element formed. T % 256 == 0.
 *   x_shared = 2: as 1, every element formed and squared even when y == NULL.
 * in % 32 == 0, out % 256 == 0, m <= 65535.
 * Replaces: archive/10M/train/val/eggroll.py:56-58 (lowrank). */
int noise_lowrank(const uint16_t* x, int32_t x_shared, const uint16_t* w, const float* noise, int64_t noise_stride,
                  int64_t a_off, int64_t b_off, const float* sign, int64_t m, int64_t T, int64_t in, int64_t out,
                  float* y, float* sumsq, void* workspace, size_t workspace_bytes, void* stream);
size_t noise_lowrank_workspace(int64_t m, int64_t T, int64_t in, int64_t out, int32_t x_shared);
/* The perturbed embedding, fp32 out [m, T, d]: out[i, t, :] = W[idx[t], :] + sign[i] a_i[idx[t]] b_i (W [vocab, d] fp32,
 * or bf16 with w_bf16 != 0; a_i = a + i a_stride [vocab], b_i = b + i b_stride [d]). d % 4 == 0, b_stride % 4 == 0,
 * m <= 65535; an id outside [0, vocab) gives a NaN row. Replaces: archive/10M/train/val/eggroll.py:61-63
 * (lowrank_embed; the population forward fuses it into its embedding kernel). */
int noise_lowrank_embed(const void* w, int32_t w_bf16, int64_t vocab, int32_t d, const float* a, int64_t a_stride,
                        const float* b, int64_t b_stride, const int64_t* idx, const float* sign, int32_t m, int64_t T,
                        float* out, void* stream);

/* The unperturbed bf16 linear of the module-by-module forward: y[r, :] = bf16(x[r, :] W^T) with fp32 accumulation,
 * x bf16 [M, in] (row stride ldx), W bf16 [out, in] (nn.Linear's weight), y bf16 [M, out] (row stride ldy).
 * in % 32 == 0, out % 256 == 0, ldx % 8 == 0, ldy % 4 == 0; x and W 16-byte aligned, y 8-byte aligned.
 * Replaces: torch.nn.Linear.forward under bf16 autocast (F.linear) for the c_q, c_k, c_v, c_proj, c_fc and lm_head
 * modules of utils/model.py:69-79, 100-104, 138 when GPT.forward runs module by module (hooked callers such as
 * train/val/dust.py:166-168). */
int noise_linear(const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t M, int64_t in, int64_t out, uint16_t* y,
                 int64_t ldy, void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): noise_lowrank's shared-x path (x_shared 1 or 2, same
 * arguments, results bit-identical to noise_lowrank's) with its workspace in a static device array of
 * NOISE_LOWRANK_STATIC_BYTES (16 MiB per GPU, held until the process ends) instead of a caller's workspace.
 * Sizes whose noise_lowrank_workspace(m, T, in, out, 1) exceeds it are rejected (NOISE_ERR_ARG); config 2 (64
 * members, T 32768, in 512, out 2048) needs 5.6 MB. Allocates nothing and records no timing events. Every call on a
 * GPU uses that GPU's one array: calls that overlap on one GPU (other streams, other host threads) race. No part of
 * the array needs to start at zero (every kernel writes what the next one reads). */
#define NOISE_LOWRANK_STATIC_BYTES (16u << 20)
int noise_lowrank_static(const uint16_t* x, int32_t x_shared, const uint16_t* w, const float* noise,
                         int64_t noise_stride, int64_t a_off, int64_t b_off, const float* sign, int64_t m, int64_t T,
                         int64_t in, int64_t out, float* y, float* sumsq, void* stream);

/* ---- a5: windowed causal attention ------------------------------------------------------------------------ */

/* out[b, t, h, :] = softmax_s(q[b,t,h] . k[b,s,h] / 8 over 0 <= t - s <= window) v[b, s, h, :]; q/k/v/out bf16 with
 * strides (batch, token) in elements and heads of 64 channels side by side (head h at +64 h); T % 128 == 0.
 * lse (optional, fp32 [batch, heads, T]) receives the log-sum-exp of each query's logits.
 * Replaces: utils/model.py:17-31 (attention / window_mask, flex_attention). */
int noise_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t batch, int32_t heads, int64_t T,
                    int64_t stride_b, int64_t stride_t, int32_t window, uint16_t* out, int64_t out_stride_b,
                    int64_t out_stride_t, float* lse, void* stream);
/* noise_attention with operands shared by groups of batch entries: with a period p > 0, batch entry e reads entry
 * e % p of that operand (0: its own), so draws stacked draw-major over a batch of p rows read one clean copy of the
 * operands they do not jitter. bounded != 0 uses the softmax without a running maximum, weights exp(s) with s = q . k / 8,
 * valid when q and k are RMS-normalized over their 64 channels (|s| <= 8). No lse output.
 * Replaces: train/val/dust.py:356-362, 372 (attention over repeat()ed operands in local_errors). */
int noise_attention_periodic(const uint16_t* q, int32_t q_period, const uint16_t* k, int32_t k_period,
                             const uint16_t* v, int32_t v_period, int64_t batch, int32_t heads, int64_t T,
                             int64_t stride_b, int64_t stride_t, int32_t window, int32_t bounded, uint16_t* out,
                             int64_t out_stride_b, int64_t out_stride_t, void* stream);

/* ---- a3, a4, a6: the perturbed population forward of the fixed GPT ---------------------------------------- */

typedef struct noise_layer {
  const uint16_t* w_qkv;      /* bf16 [1536, 512]: c_q, c_k, c_v rows stacked (nn.Linear [out, in]) */
  const uint16_t* w_proj;     /* bf16 [512, 512]  attn.c_proj */
  const uint16_t* w_fc;       /* bf16 [2048, 512] mlp.c_fc */
  const uint16_t* w_mlp_proj; /* bf16 [512, 2048] mlp.c_proj */
  const float* w_gate;        /* fp32 [8, 32] attn.ve_gate, NULL on blocks without value embeddings */
  const float* ve;            /* fp32 [padded_vocab, 512] value_embeds.{i}, NULL likewise */
  int32_t window;             /* left window of the causal attention */
} noise_layer;

typedef struct noise_gpt {
  int32_t n_layer;
  int32_t vocab;              /* logits used by the loss (GPTConfig.vocab_size) */
  int32_t padded_vocab;       /* rows of wte / lm_head / value tables, multiple of 256, at most 4096 */
  const float* resid_lambdas; /* fp32 [n_layer] */
  const float* x0_lambdas;    /* fp32 [n_layer] */
  const float* wte;           /* fp32 [padded_vocab, 512] */
  const uint16_t* lm_head;    /* bf16 [padded_vocab, 512] */
  const float* rope_cos;      /* fp32 [T, 32]: the bf16 rotary table's values (utils/model.py:177-183); the kernels
                                 read them at bf16 precision */
  const float* rope_sin;
  noise_layer layers[NOISE_MAX_LAYERS];
} noise_gpt;

/* Where each parameter's (a | b) slice (eps for the lambdas) sits in a noise row. rows == NULL: no perturbation. */
typedef struct noise_perturbation {
  const float* rows;          /* fp32 [n_rows, stride] */
  int64_t stride;
  int64_t n_rows;             /* rows of `rows` (>= 1 when rows != NULL): the range member_row is checked against */
  int64_t resid_lambdas, x0_lambdas, wte, lm_head;
  int64_t c_q[NOISE_MAX_LAYERS], c_k[NOISE_MAX_LAYERS], c_v[NOISE_MAX_LAYERS], c_proj[NOISE_MAX_LAYERS];
  int64_t ve_gate[NOISE_MAX_LAYERS], c_fc[NOISE_MAX_LAYERS], mlp_proj[NOISE_MAX_LAYERS], ve[NOISE_MAX_LAYERS];
} noise_perturbation;

/* Evaluates `members` perturbed models, member i on token row member_seq[i] with noise row member_row[i] scaled by
 * member_sign[i] (+-sigma), T tokens each (T % 128 == 0). tokens / targets int64 [n_seq, T]; a target < 0 is ignored.
 * The member tables live on the device and are checked there: a member whose member_seq is outside [0, n_seq) or
 * whose member_row is outside [0, pert->n_rows) reads nothing out of range and gets a NaN loss (every token NaN).
 * Outputs (each may be NULL): loss_sum fp32 [members] = summed next-token CE of each member; token_loss fp32
 * [members, T]; logits fp32 [members, T, vocab] (soft-capped, 15 tanh(z / 15)).
 * workspace: noise_population_forward_workspace(members, T) bytes of device memory.
 * Replaces: archive/10M/train/val/eggroll.py:66-103 (population_loss) and, with rows == NULL,
 * utils/model.py:193-210 (GPT.forward). */
size_t noise_population_forward_workspace(int64_t members, int64_t T);
int noise_population_forward(const noise_gpt* model, const noise_perturbation* pert, const int64_t* tokens,
                             const int64_t* targets, int64_t n_seq, int64_t T, const int32_t* member_seq,
                             const int32_t* member_row, const float* member_sign, int64_t members, float* loss_sum,
                             float* token_loss, float* logits, void* workspace, size_t workspace_bytes, void* stream);

/* ---- a7, a8, a9: fitness, gradient assembly, optimizer ---------------------------------------------------- */

/* fitness[j] = (L[2j+1] - L[2j]) / (std + 1e-8) with the unbiased std over j < members / 2; weight[d] = sum of
 * fitness[j] over j % pairs == d. fp32; members even.
 * Replaces: archive/10M/train/val/eggroll.py:151-154. */
int noise_fitness(const float* losses, int64_t members, int64_t pairs, float* fitness, float* weight, void* stream);

/* grad[o, i] = scale * sum_j weight[j] a_j[o] b_j[i] over j < pairs, with a_j = rows[j * stride + a_off + (0..out)],
 * b_j = rows[j * stride + b_off + (0..in)] (fp32 accumulation). 1-D parameters (b_off < 0):
 * grad[i] = scale * sum_j weight[j] rows[j * stride + a_off + i] for i < in. With accumulate != 0 the sum is added
 * to grad (grad += scale * sum), so the pairs can come in chunks of rows generated one chunk at a time.
 * Replaces: archive/10M/train/val/eggroll.py:155-166 (scale = -1 / len(fitness)). */
int noise_outer_grad(const float* rows, int64_t stride, int64_t a_off, int64_t b_off, const float* weight,
                     int64_t pairs, int64_t out, int64_t in, float scale, int32_t accumulate, float* grad, void* stream);

/* noise_outer_grad for n matrices in one launch (fp32 MFMA, 128 x 128 output tiles; each matrix j as noise_outer_grad
 * with a_off[j], b_off[j] >= 0, out[j], in[j] and grads[j], a host array of device pointers). The per-parameter loop
 * of the update becomes one grid that fills the GPU even where single matrices are small (512 x 512).
 * Replaces: archive/10M/train/val/eggroll.py:155-163 (the loop over parameters and chunks of directions). */
int noise_outer_grad_batch(const float* rows, int64_t stride, const float* weight, int64_t pairs, int32_t n,
                           const int64_t* a_off, const int64_t* b_off, const int64_t* out, const int64_t* in,
                           float* const* grads, float scale, int32_t accumulate, void* stream);

/* Dust's local linear map from a site's output error to its weight error (reassemble):
 * grad[o, i] = scale * sum_t error[t * error_ld + o] * x[t * x_ld + i] for t < tokens, o < d_out, i < d_in; x is fp32,
 * or bf16 with x_bf16 != 0 (the captured bf16 site inputs). fp32 products and sums (fp32 MFMA).
 * Replaces: train/val/dust.py:386-392 and train/val/run.py:861-867 (einsum 'btd,bti->di'). */
int noise_reassemble(const float* error, int64_t error_ld, const void* x, int32_t x_bf16, int64_t x_ld, int64_t tokens,
                     int64_t d_out, int64_t d_in, float scale, float* grad, void* stream);

/* The embedding case: grad[v, :] = sum of error[t, :] over the tokens t with ids[t] == v, for v < vocab (every row is
 * written; ids outside [0, vocab) contribute nothing). Deterministic (a fixed order per row).
 * Replaces: train/val/dust.py:389-391, train/val/run.py:864-866 (index_add_ over the token ids). */
int noise_reassemble_embedding(const float* error, int64_t error_ld, const int64_t* ids, int64_t tokens, int64_t vocab,
                               int64_t width, float* grad, void* stream);

/* One AdamW step on n fp32 elements in place (torch.optim.AdamW arithmetic): p *= 1 - lr wd; m = lerp(m, g, 1-b1);
 * v = b2 v + (1 - b2) g^2; p -= lr / (1 - b1^step) * m / (sqrt(v) / sqrt(1 - b2^step) + eps).
 * shadow (optional): bf16 copy of the updated p. Replaces: archive/10M/train/val/eggroll.py:205, 167 and
 * train/speedrun/run.py:2866-2883 (_adamw_kernel). */
int noise_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                float eps, float weight_decay, int64_t step, uint16_t* shadow, void* stream);

/* noise_adamw over n tensors with shared hyperparameters and step in one launch per 48 tensors (host arrays of
 * device pointers and sizes; shadow may be NULL, or an array whose entries may be NULL). p, g, m and v 16-byte
 * aligned, bf16 copies 8-byte aligned. Replaces: torch.optim.AdamW.step over a parameter group
 * (archive/10M/train/val/eggroll.py:205, 167; its foreach path) and train/speedrun/run.py:2866-2916 (the fused
 * multi-tensor _adamw_kernel launch). */
int noise_adamw_batch(int32_t n, float* const* p, const float* const* g, float* const* m, float* const* v,
                      uint16_t* const* shadow, const int64_t* numel, float lr, float beta1, float beta2, float eps,
                      float weight_decay, int64_t step, void* stream);

/* ---- a10, a11, a12: cross-token credit readout ------------------------------------------------------------ */

/* lse[r, s] = log sum_{t in [s - window, s]} exp(q[r, s] . k[r, t] / 8); q, k bf16 [rows, T, 64], T % 128 == 0,
 * rows <= 65535. The lse alone, for callers that need no center (train/val/run.py:965-985 builds A from it).
 * Replaces: train/speedrun/moment_kernels.py:79-110, 137-164 (_implicit_key_statistics, its lse output). */
int noise_credit_lse(const uint16_t* q, const uint16_t* k, int64_t rows, int64_t T, int32_t window, float* lse,
                     void* stream);
/* noise_credit_lse for callers whose logits are bounded, |q . k| / 8 <= 16 on every in-window pair (q and k
 * RMS-normalized over their 64 channels give <= 8, as the model's do): the sum of exp(logit) then stays inside fp32
 * with no running maximum at any T and window (e^16 times 2^31 terms is below 2^128), and each logit costs one exp2
 * (q carries the scale log2(e) / 8: one more bf16 rounding of q, which moves a logit by at most 16 * 2^-9 = 0.03 at
 * the bound). Larger logits lose accuracy and, near 88, overflow the sum (lse inf or NaN). Same arguments and errors
 * as noise_credit_lse.
 * Replaces: train/speedrun/moment_kernels.py:79-110 (_implicit_key_statistics' lse) where its inputs are bounded. */
int noise_credit_lse_bounded(const uint16_t* q, const uint16_t* k, int64_t rows, int64_t T, int32_t window,
                             float* lse, void* stream);
/* The key context of each receiver s: lse[r, s] as noise_credit_lse, and
 * center[r, s] = sum_{t in [s - window, s]} exp(q[r, s] . k[r, t] / 8 - lse[r, s]) (hub[r, s] . values[r, t]),
 * the softmax-weighted mean of the value scores. q, k, values, hub bf16 [rows, T, 64]; fp32 probabilities and
 * accumulation; T % 128 == 0, rows <= 65535.
 * Replaces: train/speedrun/moment_kernels.py:79-110 (_implicit_key_statistics), 137-164 (the _edges variant, same
 * outputs up to summation order), 167-194 (_implicit_key_context / implicit_key_context_edges). */
int noise_credit_key_context(const uint16_t* q, const uint16_t* k, const uint16_t* values, const uint16_t* hub,
                             int64_t rows, int64_t T, int32_t window, float* lse, float* center, void* stream);

/* out[r, t, :] = sum_{s in [t, t + window]} exp(k[r, t] . q[r, s] / 8 - lse[r, s]) src[r, s, :]; src fp32
 * [rows, T, 64] used as its bf16 high part (hi_lo != 0: high + low parts), probabilities in bf16, fp32 accumulation.
 * Replaces: train/speedrun/moment_kernels.py:612-661 (_value_credit_kernel / _value_pass) and
 * train/speedrun/value_gluon.py:145-172 (value_pass_gluon). */
int noise_credit_value(const uint16_t* q, const uint16_t* k, const float* lse, const float* src, int64_t rows,
                       int64_t T, int32_t window, int32_t hi_lo, float* out, void* stream);
/* noise_credit_value with _value_pass's layouts handled in the kernel: q, k (rows, T, 64) and lse (rows, T) stacked as
 * above; the source row r at head r % src_heads of token row r / src_heads (fp32, row stride src_sb, token stride
 * src_st, heads of 64 side by side); the output row r written at head r % out_heads of output row
 * out_rows[r / out_heads] (r / out_heads when out_rows is NULL; row stride out_sb, token stride out_st). src_heads and
 * out_heads divide rows; strides in elements, multiples of 4. out_rows (device int32, rows / out_heads entries) must
 * index rows of out: the kernel does not check them.
 * Replaces: train/speedrun/moment_kernels.py:645-661 (_value_pass with in_heads, out_heads, out and layers; the
 * by-token row order of _by_token, :67-74). */
int noise_credit_value_strided(const uint16_t* q, const uint16_t* k, const float* lse, const float* src,
                               int32_t src_heads, int64_t src_sb, int64_t src_st, int64_t rows, int64_t T,
                               int32_t window, int32_t hi_lo, float* out, int32_t out_heads, int64_t out_sb,
                               int64_t out_st, const int32_t* out_rows, void* stream);

/* ---- next rows: Dust's direct draws and head-slab CE estimator ----------------------------------------------- */

/* One chunk of direct draws (train/val/dust.py:210-259): n_draws draws of the batch's n_seq sequences, member m =
 * (draw draw0 + m / n_seq, batch row m % n_seq), each adding sigma a (this library's counter-based Gaussians, by seed,
 * draw, site and token row) at the chosen sites of block `entry` and rerunning the network from there. */
typedef struct noise_dust_draws {
  int32_t entry;      /* the jittered block; -1: the token embedding (every block reruns, from the embedding) */
  const float* x_in;  /* entry >= 0: fp32 [n_seq, T, 512], the captured (mixed) input of block `entry` */
  const float* x0_in; /* entry >= 0: fp32 [n_seq, T, 512], the captured x0 = norm(embedding) */
  int32_t sites;      /* bit s jitters site s: 0 the token embedding (entry -1); 1 the attention output (before
                         attn.c_proj), 2 attn.c_proj's output, 3 mlp.c_fc's output, 4 mlp.c_proj's output */
  float sigma;
  uint64_t seed;
  int32_t draw0;      /* global index of the chunk's first draw (the jitter stream's draw counter) */
  int32_t n_draws;
} noise_dust_draws;

/* The clean pass (dust.py:195-208, DUST.capture): token_loss fp32 [n_seq, T] (per-token CE, 0 where targets == -1) and
 * capture fp32 [n_layer + 1, n_seq, T, 512]: the mixed input of every block (the blocks' forward pre-hooks), then x0.
 * tokens, targets int64 [n_seq, T]; T % 128 == 0. Workspace: noise_dust_workspace(1, n_seq, T).
 * Replaces: train/val/dust.py:176-208 (the capture hooks and DUST.capture's clean losses). */
int noise_dust_capture(const noise_gpt* model, const int64_t* tokens, const int64_t* targets, int64_t n_seq,
                       int64_t T, float* token_loss, float* capture, void* workspace, size_t workspace_bytes,
                       void* stream);

/* noise_dust_capture that also keeps, per block, the inputs of the writers' linears (each pointer may be NULL):
 * attn_in [n_layer, n_seq * T, 512] bf16 attn.c_proj's input (the attention output); fc_in [n_layer, n_seq * T, 512]
 * fp32 mlp.c_fc's input (the MLP's RMS-normed input); mlp_in [n_layer, n_seq * T, 2048] bf16 mlp.c_proj's input
 * (relu² of c_fc). They hold the values the reference's hooks cache (the bf16 activations are exact in bf16), and are
 * what noise_reassemble multiplies a site's output error by.
 * Replaces: train/val/dust.py:139-179 (the forward hooks caching every Linear's input, self.inputs). */
int noise_dust_capture_sites(const noise_gpt* model, const int64_t* tokens, const int64_t* targets, int64_t n_seq,
                             int64_t T, float* token_loss, float* capture, uint16_t* attn_in, float* fc_in,
                             uint16_t* mlp_in, void* workspace, size_t workspace_bytes, void* stream);
/* Per-token CE of the chunk's draws, token_loss fp32 [n_draws, n_seq, T], clean weights.
 * Workspace: noise_dust_workspace(n_draws, n_seq, T).
 * Replaces: train/val/dust.py:210-233 (DUST.rerun with block_forward's jitter sites, :104-120, and head_loss,
 * :94-99), its torch.randn jitter (:192-193, 244) replaced by the counter stream. */
int noise_dust_rerun(const noise_gpt* model, const noise_dust_draws* draws, const int64_t* tokens,
                     const int64_t* targets, int64_t n_seq, int64_t T, float* token_loss, void* workspace,
                     size_t workspace_bytes, void* stream);
size_t noise_dust_workspace(int64_t n_draws, int64_t n_seq, int64_t T);
/* One chunk's contribution to a site's error estimate (dust.py:246-257): reward[j] = clean_loss - token_loss[j],
 * centered over the chunk's draws when n_draws > 1, then (gamma > 0) the decayed reward-to-go along T (dust.py:86-91);
 * error fp32 [n_seq, T, width] -= sum_j reward[j] a_j / sigma, with a_j the draw's jitter at `site` regenerated from
 * (seed, draw0 + j). The caller zeroes error before a site's first chunk and divides by the draw count after the last.
 * Workspace: noise_dust_errors_workspace(n_draws, n_seq, T).
 * Replaces: train/val/dust.py:235-259 (DUST.direct_errors' reward and einsum). */
int noise_dust_errors(const float* token_loss, const float* clean_loss, int32_t n_draws, int64_t n_seq, int64_t T,
                      float gamma, float sigma, uint64_t seed, int32_t draw0, int32_t site, int32_t width,
                      float* error, void* workspace, size_t workspace_bytes, void* stream);
size_t noise_dust_errors_workspace(int32_t n_draws, int64_t n_seq, int64_t T);


/* error[r, v] (fp32 [b * t, ld], rows r = bi * t + ti) = per-token error estimates of the lm_head outputs raw (bf16
 * [b * t, ld], the clean forward's, before the soft cap): chunk c of n draws (n = the largest count <= nrep that
 * divides draws) jitters vocabulary slab c % (vocab / 256) by sigma a (this library's counter-based Gaussians,
 * streamed by seed, draw and row), recomputes each token's soft-capped CE from the cached sums of the other slabs,
 * rewards clean_loss - CE (0 where targets == -1; centered over the batch when b > 1), and error of the slab's columns
 * = -(sum over its draws of reward / sigma * a) / (draws per slab); columns from vocab to ld are 0.
 * vocab % 256 == 0, vocab <= ld, ld % 4 == 0, (draws / n) % (vocab / 256) == 0, draws <= 65535, b * t <= 2^26.
 * Workspace: noise_head_error_workspace(b * t, vocab, draws) bytes.
 * Replaces: train/val/dust.py:261-303 (DUST.head_error), with its torch.randn jitter (dust.py:192-193) replaced by the
 * counter stream. */
int noise_head_error(const uint16_t* raw, int64_t ld, const int64_t* targets, const float* clean_loss, int32_t b,
                     int32_t t, int32_t vocab, int32_t draws, int32_t nrep, float sigma, uint64_t seed, float* error,
                     void* workspace, size_t workspace_bytes, void* stream);
size_t noise_head_error_workspace(int64_t rows, int32_t vocab, int32_t draws);

/* Decayed credit of later tokens' scores, fp32: for each row (o, i) of a [outer, T, inner] array,
 * out[o, t, i] = sum_{s = t}^{min(t + window, T - 1)} gamma^(s - t) score[o, s, i], in O(T) per row (no T x T matrix).
 * out may be score itself. T % 256 == 0, T <= 8192, window >= 0, 0 < gamma < 1, outer * inner < 2^31.
 * Replaces: train/val/dust.py:342-345 (the [T, T] credit matrix [0 <= s - t <= window] gamma^(s - t)) and :378-381
 * (its einsum 'nbsh,ts->nbth' with the per-head scores: outer = n * b, inner = heads). */
int noise_decayed_credit(const float* score, int64_t outer, int64_t T, int32_t inner, int32_t window, float gamma,
                         float* out, void* stream);
/* The local draws' jitter, fp32 [n_draws, rows, width]: draw draw0 + d at `site`, element (row, c) from the counter
 * stream that the direct draws' jitter uses (seed, draw, site, row), so a site id outside the direct draws' 0..4 keys
 * an independent stream. width % 4 == 0, n_draws <= 65535.
 * Replaces: train/val/dust.py:349 (self.noise(n, b, t, width), torch.randn on the estimator's generator). */
int noise_dust_noise(uint64_t seed, uint32_t draw0, uint32_t site, int32_t n_draws, int64_t rows, int32_t width,
                     float* out, void* stream);
/* The local draws' jittered operand, bf16 [n_draws * b * t, 512] (rows (j b + bi) t + tt, 8 heads of 64): with a_j
 * draw draw0 + j of the counter stream at `site` (as noise_dust_noise, 512 wide; 8 wide for the gate),
 *   kind 0 (q, k):  norm(rotary(raw + sigma a_j)) per head, raw bf16 [b * t, 512], cos / sin fp32 [t, 32]
 *   kind 1 (v):     sigma a_j
 *   kind 2 (ve):    sigma a_j 2 sigmoid(z_h), z bf16 [b * t, 8]
 *   kind 3 (gate):  (2 sigmoid(z_h + sigma a_jh) - 2 sigmoid(z_h - sigma a_jh)) ve, ve fp32 [b * t, 512]
 * Replaces: train/val/dust.py:349-372 (the jitter, processed() and the jittered values of local_errors). */
int noise_local_operand(int32_t kind, uint64_t seed, uint32_t draw0, uint32_t site, int32_t n_draws, int32_t b,
                        int32_t t, const uint16_t* raw, const uint16_t* z, const float* ve, const float* cos_table,
                        const float* sin_table, float sigma, uint16_t* out, void* stream);
/* score fp32 [n_draws * b * t, 8]: per head, the sum over its 64 channels of target[bi, tt] (fp32 [b * t, 512]) times
 * att[row] - baseline[bi, tt] (bf16; baseline NULL: att itself).
 * Replaces: train/val/dust.py:356-362, 375-377 (the output change and einsum 'bthd,nbthd->nbth'). */
int noise_local_score(const uint16_t* att, const uint16_t* baseline, const float* target, int32_t n_draws, int32_t b,
                      int32_t t, float* score, void* stream);
/* err fp32 [b * t, width] += inv_divisor * sum_j score[(j b + bi) t + tt, head] a_j[bi, tt, c] over the chunk's draws,
 * the jitter regenerated from the counter stream (width 512; 8 for the gate, where the channel is the head).
 * Replaces: train/val/dust.py:378-382 (einsum 'nbth,nbthd->bthd' and the division by the divisor). */
int noise_local_estimate(const float* score, uint64_t seed, uint32_t draw0, uint32_t site, int32_t n_draws, int32_t b,
                         int32_t t, int32_t width, float inv_divisor, float* err, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NOISE_AMD_H */
