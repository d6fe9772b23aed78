/* Decode-step pieces of the hybrid models on gfx950 (workloads C4 and C5).
 *
 * C4 is Qwen3.5-35B-A3B-style (gated DeltaNet + GQA layers, softmax-top-8 MoE);
 * its arithmetic follows the reference example's plain-torch twin
 * (examples/qwen3_5_35b_a3b-tilelang/kernels/torch_ref.py:22-40: f32 activations
 * and state, matmuls at the weights' bf16 with one rounding of the f32 sum).
 * C5 is Granite-4.0-H-style (Mamba2 + GQA layers, top-10-then-softmax MoE) with
 * fp8-e4m3fn weights and per-output-channel f32 scales; its arithmetic follows
 * the authored HIR (examples/granite_4_0_h_small-cuda/model.py: bf16 ops rounded
 * as written, f32 where it casts to f32).
 *
 * Every entry returns 0 or an error (tfd_last_error() holds the text), takes
 * device pointers and a hipStream_t, allocates nothing and does not synchronise.
 * Batch rows are sequences, one token each.  The projections around these
 * entries are tfd_gemm_skinny_bf16 / tfd_gemm_skinny_fp8 (tf_decode.h); GEMM
 * inputs are in the skinny GEMMs' operand order (tf_decode.h). */
#ifndef TF_HYBRID_H
#define TF_HYBRID_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp8-e4m3fn weights with one f32 scale per output row (workload C5's
 * "fp8 per-channel" projections).  The reference has no fp8 GEMV: its Granite
 * projections are bf16 nn.Linear (examples/granite_4_0_h_small-cuda/
 * model.py:140-152 in_projection, :266-270 out_proj, :294-330 attention
 * q/k/v/o, :459-471 shared MLP), so this build
 * defines W[n][k] = f32(e4m3fn(code[n][k])) * scale[n].
 * tfd_pack_skinny_fp8 lays codes [N][K] (row stride ldw bytes) out in 512-byte
 * blocks of 16 rows x 32 k, the fp8 counterpart of tfd_pack_skinny_bf16; `packed`
 * holds ceil(N/16) * 16 * K bytes.  K % 256 == 0. */
int tfd_pack_skinny_fp8(const void* w, int ldw, int N, int K, void* packed, void* stream);

/* Y[m][n] = scale[n] * sum_k X[m][k] e4m3(W[n][k]) for m < M <= 32 (f32 sums,
 * one bf16 rounding per output), X in operand order, W packed by
 * tfd_pack_skinny_fp8, scale f32 [N]; the epilogues of tfd_gemm_skinny_bf16.
 * K splits across the waves of one block (no work buffer). */
int tfd_gemm_skinny_fp8(const void* x, const void* w, const float* scale, int M, int K, int N,
                        int epilogue, const void* resid, int ldr, void* out, int ldo,
                        void* stream);
/* The same product with C5's scaled residual add as its epilogue: out =
 * bf16(resid + bf16(y * mult)), y the bf16 product (examples/granite_4_0_h_small-cuda/
 * model.py:502-508 residual_add after the mixer's out_proj).  out may alias resid. */
int tfd_gemm_skinny_fp8_resid_scaled(const void* x, const void* w, const float* scale, int M,
                                     int K, int N, const void* resid, int ldr, float mult,
                                     void* out, int ldo, void* stream);

/* The HIR's rms_norm op on each of `rows` bf16 vectors of n values: out =
 * bf16(f32(f32(x * rsqrt(mean(x^2) + eps)) * gamma)), one rounding (the evaluator's
 * handler, src/tilefoundry/ir/hir/nn/rms_norm.py:103-110).  The Granite model writes
 * its input, post-mixer and final norms this way (examples/granite_4_0_h_small-cuda/
 * model.py:149, 291, 403, 632); the Qwen3 norm (tfd_rmsnorm_rows_bf16) rounds before
 * gamma instead.  Written row-major to out_rows [rows][ldo] and/or in the skinny GEMMs'
 * operand order to out_packed (rows <= 32, n % 32 == 0); NULL skips one. */
int tfd_tf_rmsnorm_rows_bf16(const void* x, int ldx, const void* gamma, void* out_rows, int ldo,
                             void* out_packed, int rows, int n, float eps, void* stream);

/* The head over a published divisor: out (f32 [M][ldo]) = bf16(bf16(x . W[n]) / divisor),
 * the product as tfd_gemm_skinny_bf16's TFD_EPI_LOGITS and its work buffer rules.
 * Replaces Granite4_0_H_Small.lm_head's `logits / logits_scaling`
 * (examples/granite_4_0_h_small-cuda/model.py:636-645). */
int tfd_gemm_skinny_bf16_logits_div(const void* x, const void* w, int M, int K, int N,
                                    float divisor, void* out, int ldo, float* work,
                                    int64_t work_floats, void* stream);

#define TFD_ROUTE_SOFTMAX_TOPK 0 /* C4: softmax over all experts, top k, renormalise */
#define TFD_ROUTE_TOPK_SOFTMAX 1 /* C5: top k logits, softmax over them, bf16 weights */

/* The routers after their projection: logits f32 [rows][ldl] (experts <= 256)
 * -> weights f32 [rows][k] (C5: bf16 values) and expert ids int32 [rows][k],
 * largest first with ties to the lower id (torch.topk's order).
 * Replaces Qwen3_5Router.routing's softmax/topk/renormalise
 * (tests/models/qwen3_5_35b_a3b/model.py:355-366; torch_ref.py:417-430) and
 * GraniteRouter.routing's topk/softmax
 * (examples/granite_4_0_h_small-cuda/model.py:376-390).
 * The reference returns int64 ids; these are int32. */
int tfd_route_topk(const float* logits, int ldl, int rows, int experts, int k, int mode,
                   float* weights, int32_t* idx, void* stream);

#define TFD_POLICY_F32 0  /* C4 (torch_ref policy) */
#define TFD_POLICY_BF16 1 /* C5 (HIR policy) */

/* Routed experts + shared expert of the MoE block for a batch, given the
 * routing (replaces Qwen3_5MoE.routed_experts/shared_expert/experts,
 * tests/models/qwen3_5_35b_a3b/model.py:383-456 / torch_ref.py:451-530, and
 * GraniteMoE.routed_experts/shared_mlp/experts, granite model.py:406-471).
 * Grouped by expert: each weight row of a picked expert is read once per call
 * however many sequences picked it.
 * Weights keep the reference's (out, in) rows: w_gate/w_up [E][I][H], w_down
 * [E][H][I]; the shared expert's gate rows then up rows in w_shared_in [2 IS][H]
 * and w_shared_out [H][IS].  With fp8 != 0 every weight is e4m3fn bytes with an
 * f32 scale per row (s_*).  C4's shared expert has a sigmoid gate row
 * w_shared_scale [H] (bf16, NULL for C5).  x [rows][H] bf16 (the post-norm
 * tokens); idx holds k distinct experts per row; out f32 [rows][H] (C5: bf16
 * values).  Work: hidden bf16 [rows][k + 1][hidden_ld], shared_scale f32 [rows],
 * partial f32 [rows][k + 1][H], groups int32 [TFD_MOE_GROUP_WORDS(experts, rows)].
 * experts <= 256, H <= 4096 and I, IS <= 2048, multiples of 64.  An expert id
 * outside [0, experts) (it is served as expert 0) or an expert repeated in a row
 * raises TFD_ERR_TOKEN_RANGE in err. */
#define TFD_MOE_GROUP_WORDS(experts, rows) (1 + 2 * (experts) + (experts) * (rows))
#define TFD_MOE_ROUTE_GIVEN 0
#define TFD_MOE_ROUTE_SOFTMAX_TOPK 1 /* TFD_ROUTE_SOFTMAX_TOPK inside the call */
#define TFD_MOE_ROUTE_TOPK_SOFTMAX 2 /* TFD_ROUTE_TOPK_SOFTMAX inside the call */
typedef struct {
  const void* x;
  const float* weights;
  const int32_t* idx;
  const void *w_gate, *w_up, *w_down;
  const float *s_gate, *s_up, *s_down;
  const void *w_shared_in, *w_shared_out;
  const float *s_shared_in, *s_shared_out;
  const void* w_shared_scale;
  void* hidden;
  float* shared_scale;
  float* partial;
  int32_t* groups;
  float* out;
  int rows, k, experts, hidden_size, inter, shared_inter, hidden_ld;
  int fp8, policy;
  int accumulate; /* TFD_POLICY_F32 only: out += the block's output (C4's residual add) */
  /* route TFD_MOE_ROUTE_SOFTMAX_TOPK / _TOPK_SOFTMAX: the call routes first, as
   * tfd_route_topk would, from logits f32 [rows][ldl] into weights / idx (then
   * outputs, k <= 64); TFD_MOE_ROUTE_GIVEN (0): weights and idx are inputs. */
  const float* logits;
  int ldl, route;
  int32_t* err;
  /* TFD_POLICY_BF16 only: with resid set, the call adds its output into the bf16
   * residual stream resid [rows][hidden_size] as resid = bf16(resid + bf16(y *
   * resid_mult)) (examples/granite_4_0_h_small-cuda/model.py:502-508
   * residual_add) instead of writing out (which may then be NULL). */
  void* resid;
  float resid_mult;
} TfdMoeArgs;
int tfd_moe_experts(const TfdMoeArgs* args, void* stream);

/* tfd_moe_experts over packed weights for rows <= 16, on the matrix cores, in
 * three launches (routing + grouping, gate/up, down + mix); same arguments and
 * outputs (partial is not used and may be NULL).  Each weight matrix is packed
 * as tfd_pack_skinny_bf16 / tfd_pack_skinny_fp8 pack a [rows][K] matrix, the
 * experts' matrices stacked: w_gate and w_up as one [E I][H] matrix each, w_down
 * as [E H][I], w_shared_in as [2 IS][H], w_shared_out as [H][IS]; the row scales
 * keep their order.  Needs k <= 16, H a multiple of 1024, I and IS multiples of
 * 256, IS <= 2048 and rows (k + 1) I / 256 <= 1024 (kBadShape otherwise).  The
 * sums of the products run in another order than tfd_moe_experts' (MFMA
 * accumulators over K instead of lane sums), so results agree to the f32
 * rounding of each sum before its bf16 rounding. */
int tfd_moe_experts_packed(const TfdMoeArgs* args, void* stream);

/* An fp8 projection of C5 with the HIR's RMSNorm as its prologue (replaces
 * GraniteDecoderLayer's input_layernorm / post_attention_layernorm followed by
 * the in-projection or the router, examples/granite_4_0_h_small-cuda/
 * model.py:480-523 with rms_norm at ir/hir/nn/rms_norm.py:103-110): for rows
 * <= 8 and K = 4096, xn = bf16(x * rsqrt(mean(x^2) + eps) * gamma) from the bf16
 * rows x [rows][ldx] (f32 arithmetic, one rounding), then out[r][n] =
 * bf16(scale[n] sum_k xn[r][k] e4m3(W[n][k])) with W packed by
 * tfd_pack_skinny_fp8: TFD_EPI_STORE bf16 [rows][ldo], TFD_EPI_LOGITS f32 (bf16
 * values) [rows][ldo].  With x_rows set the normalised rows are also written
 * there ([rows][ldxr] bf16: the experts' input).  One launch instead of a norm
 * and a GEMM; kBadShape outside those sizes. */
typedef struct {
  const void* x;
  int ldx;
  const void* gamma;
  float eps;
  void* x_rows;
  int ldxr;
  const void* w;
  const float* scale;
  int rows, K, N;
  void* out;
  int ldo, epilogue;
} TfdProj8NormArgs;
int tfd_proj8_norm(const TfdProj8NormArgs* args, void* stream);

/* Gated DeltaNet at one token per sequence, everything between the in- and
 * out-projections of Qwen3_5LinearAttention.linear_attention: conv_step,
 * l2_normalise, beta/g, delta_step and the gated RMS norm
 * (tests/models/qwen3_5_35b_a3b/model.py:124-232; torch_ref.py:188-312).  proj
 * f32 [rows][proj_ld] holds this token's projections (bf16 values): the conv
 * channels q|k|v (2 hk dk + hv dv), then z (hv dv), b (hv), a (hv).
 * conv_in/conv_out f32 [rows][CONV][3] (distinct
 * buffers: the window after this token goes to conv_out); state f32
 * [rows][hv][dk][dv] is updated in place.  out: the gated read-out in operand
 * order (32 x hv dv) for the out-projection.  dk = dv = 128, conv kernel 4. */
typedef struct {
  const float* proj;
  int proj_ld;
  const float* conv_in;
  float* conv_out;
  float* state;
  const void *conv_w, *a_log, *dt_bias, *gamma;
  void* out;
  int rows, key_heads, value_heads, head_k_dim, head_v_dim, conv_kernel;
  float l2_eps, rms_eps;
} TfdGdnArgs;
int tfd_gdn_step(const TfdGdnArgs* args, void* stream);

/* Mamba2 at one token per sequence, everything between in_proj and out_proj of
 * GraniteMamba.mamba_mixer: conv_step, ssm_step and gated_out's RMSNormGated
 * (examples/granite_4_0_h_small-cuda/model.py:154-270).  proj bf16 [rows][proj_ld]: gate
 * (EXP), the conv channels x|B|C (EXP + 2 ns), dt (heads); conv_in/conv_out bf16
 * [rows][CONV][3] (distinct); state f32 [rows][heads][64][128] in place.  Work:
 * gated f32 [rows][EXP], ssq f32 [rows][heads].  out: the normed gated output in
 * operand order (32 x EXP) for out_proj.  head_dim 64, state 128, 1 group. */
typedef struct {
  const void* proj;
  int proj_ld;
  const void* conv_in;
  void* conv_out;
  float* state;
  const void *conv_w, *conv_b, *a_log, *dt_bias, *d_skip, *gamma;
  float* gated;
  float* ssq;
  void* out;
  int rows, heads, head_dim, state_dim, groups, conv_kernel;
  float eps;
} TfdMambaArgs;
int tfd_mamba_step(const TfdMambaArgs* args, void* stream);

/* The full-attention layers of both hybrids at one token per sequence,
 * between the q/k/v projections and o_proj: GQA decode over the paged bf16 KV
 * cache of tf_decode.h ([pages][kv_heads][16][head_dim], 16 positions a page),
 * after appending this token's key and value at pos[b].
 *  policy TFD_POLICY_F32 (C4, Qwen3_5FullAttention.full_attention,
 *    tests/models/qwen3_5_35b_a3b/model.py:234-346 / torch_ref.py:318-409):
 *    qkv f32 [rows][ldq] (bf16 values) holds per
 *    query head its query then its output gate (2 head_dim each), then the keys,
 *    then the values; per-head RMSNorm (gamma_q, gamma_k, flat), rotate-half
 *    RoPE on the first rot_dim dims (cos/sin bf16 [rope_rows][rot_dim]), query
 *    times `scale`, softmax, output times sigmoid(gate); all f32; the cache keeps
 *    bf16(k_rope).  head_dim 256, 8 query heads per kv head.
 *  policy TFD_POLICY_BF16 (C5, GraniteAttention.attend after cache_update,
 *    examples/granite_4_0_h_small-cuda/model.py:310-366):
 *    qkv bf16 [rows][ldq] = queries, keys, values; no
 *    position embedding; score = bf16(sum bf16(q k)) * scale in f32, softmax f32
 *    rounded to bf16, attn = bf16(sum bf16(p v)).  head_dim 128, 4 query heads per
 *    kv head.  gamma/cos/sin unused.
 * out: o_proj's input in operand order (32 x heads * head_dim bf16).  Work:
 * scores f32 [rows][heads][score_stride >= max_pages * 16], stats f32
 * [rows][heads][nsplit][2], part f32 [rows][heads][nsplit][head_dim], counters
 * int32 [rows][kv_heads] (zero; left zero).  A split covers split_len positions
 * (a multiple of 16, <= 512); nsplit * split_len >= max_pages * 16.  split_len 0:
 * each row's split length follows its position, ceil((pos + 1) / nsplit) rounded up
 * to 16, between 64 and 512 (nsplit * 512 >= max_pages * 16).  A position
 * outside the page (or rope) table raises TFD_ERR_POS_RANGE in err, a page
 * outside the pool TFD_ERR_PAGE_RANGE. */
typedef struct {
  const void* qkv;
  int ldq;
  const void *gamma_q, *gamma_k, *cos_table, *sin_table;
  int rope_rows, rot_dim;
  const int32_t* pos;
  const int32_t* page_table;
  int max_pages;
  void *k_pool, *v_pool;
  int num_pages;
  int rows, heads, kv_heads, head_dim;
  float scale, eps;
  float* scores;
  int score_stride;
  float* stats;
  float* part;
  int32_t* counters;
  int nsplit, split_len;
  void* out;
  int policy;
  int32_t* err;
} TfdGqaArgs;
int tfd_gqa_decode(const TfdGqaArgs* args, void* stream);

/* C4's f32 residual stream (torch_ref.py's policy: activations f32, a matmul
 * casts its input to bf16).  tfd_rmsnorm_f32_rows: out = bf16(x * rsqrt(mean(x^2)
 * + eps) * gamma) per row, f32 inside and one rounding (torch_ref.py:145-154
 * `_rms_norm` followed by `_mm`'s cast; input_layernorm, post_norm :438-448 and
 * final_rms_norm :558-567), to row-major out_rows [rows][ldo] and/or out_packed in
 * the skinny GEMMs' operand order (rows <= 32, n % 32 == 0); NULL skips one.
 * tfd_add_f32_rows: acc += add (residual_add, :533-543).  tfd_bf16_to_f32_rows:
 * dst = f32(src) (embed's `.float()` of the table row, :546-555). */
int tfd_rmsnorm_f32_rows(const float* x, int ldx, const void* gamma, void* out_rows, int ldo,
                         void* out_packed, int rows, int n, float eps, void* stream);
int tfd_add_f32_rows(float* acc, int lda, const float* add, int ldb, int rows, int n,
                     void* stream);
int tfd_bf16_to_f32_rows(const void* src, int lds, float* dst, int ldd, int rows, int n,
                         void* stream);

/* C5's scaled residual and embedding (examples/granite_4_0_h_small-cuda/
 * model.py:502-508 residual_add, :615-624 embed): out = bf16(a + bf16(b * m)) per
 * element, a NULL `a` giving bf16(b * m); b is bf16 [rows][ldb], or f32 holding
 * bf16 values with b_f32 != 0 (the experts' output).  out may alias a. */
int tfd_scaled_add_rows(const void* a, int lda, const void* b, int ldb, int b_f32, float m,
                        void* out, int ldo, int rows, int n, void* stream);

/* The mixers' authored sub-functions, one launch each, for the runtime twins
 * (tilefoundry_amd/hybrid/twin.py) -- the decode engines run the fused
 * tfd_gdn_step / tfd_mamba_step instead, with the same arithmetic.  One token per
 * row; no work buffers.
 *
 * tfd_conv_step_rows: the depthwise causal convolution closing on this token,
 * out[c] = silu(sum_t window[c][t] * w[c][t] (+ bias[c])) over the 3-tap window
 * [rows][channels][3] and the entry [rows][lde] (conv kernel 4).  policy
 * TFD_POLICY_F32: f32 window / entry / out, no bias (Qwen3_5LinearAttention.
 * conv_step, tests/models/qwen3_5_35b_a3b/model.py:124-136); TFD_POLICY_BF16: bf16
 * window / entry / out, every product, the sum and the biased value rounded to bf16
 * (GraniteMamba.conv_step, examples/granite_4_0_h_small-cuda/model.py:154-168). */
typedef struct {
  const void* window;
  const void* entry;
  int lde;
  const void *conv_w, *conv_b; /* bf16 [channels][4], bf16 [channels] or NULL */
  void* out;
  int ldo, rows, channels, kernel, policy;
} TfdConvStepArgs;
int tfd_conv_step_rows(const TfdConvStepArgs* args, void* stream);

/* Qwen3_5LinearAttention.l2_normalise (model.py:138-146): out = x * rsqrt(sum(x^2) +
 * eps) for each of nvec f32 vectors of dim <= 256 (out may alias x). */
int tfd_l2norm_f32(const float* x, float* out, int nvec, int dim, float eps, void* stream);

/* Qwen3_5LinearAttention.delta_step (model.py:148-172) on an f32 state: with
 * decay = exp(g), recalled = sum_k decay S[k][:] k[k], delta = (v - recalled) beta,
 * S' = decay S + k delta^T, read = sum_k S'[k][:] q[k] qscale.  state_in/state_out
 * [rows][heads][128][128] (may alias), q/k [rows][heads][128], v [rows][heads][128],
 * g/beta [rows][heads], read [rows][heads][128], all f32. */
typedef struct {
  const float* state_in;
  float* state_out;
  const float *q, *k, *v, *g, *beta;
  float* read;
  float qscale;
  int rows, heads, head_k_dim, head_v_dim;
} TfdDeltaStepArgs;
int tfd_delta_step_f32(const TfdDeltaStepArgs* args, void* stream);

/* Qwen3_5FullAttention.partial_rope / partial_rope_kv (model.py:235-262, torch_ref
 * f32): the first rot dims of each head as x * cos + rotate_half(x) * sin with the
 * bf16 table rows at pos[row] ([rope_rows][rot]), the rest copied.  x / out f32
 * [rows][ld] holding heads x head_dim values. */
typedef struct {
  const float* x;
  int ldx;
  float* out;
  int ldo;
  const int32_t* pos;
  const void *cos_table, *sin_table;
  int rope_rows, rows, heads, head_dim, rot;
} TfdPartialRopeArgs;
int tfd_partial_rope_f32(const TfdPartialRopeArgs* args, void* stream);

/* GraniteMamba.ssm_step (examples/granite_4_0_h_small-cuda/model.py:170-221) at the
 * HIR's bf16 rounding: dt = softplus(dt_raw + dt_bias), decay = exp(dt * -exp(a_log)),
 * S' = S decay + bf16(bf16(dt B) x), y = bf16(C . bf16(S')) + bf16(x D).  state_in /
 * state_out f32 [rows][heads][64][128] (may alias); x bf16 [rows][ldx] (heads x 64),
 * b_vec / c_vec bf16 [rows][ld] (128, one group), dt_raw bf16 [rows][lddt],
 * a_log / dt_bias / d_skip bf16 [heads]; y bf16 [rows][ldy]. */
typedef struct {
  const float* state_in;
  float* state_out;
  const void* x;
  int ldx;
  const void* b_vec;
  int ldb;
  const void* c_vec;
  int ldc;
  const void* dt_raw;
  int lddt;
  const void *a_log, *dt_bias, *d_skip;
  void* y;
  int ldy, rows, heads, head_dim, state_dim;
} TfdSsmStepArgs;
int tfd_ssm_step_bf16(const TfdSsmStepArgs* args, void* stream);

/* gated_out's RMSNormGated (model.py:223-237): g = f32(y) * silu(f32(gate)), out =
 * bf16(g * rsqrt(mean(g^2) + eps) * gamma) per row of n <= 8192 (y, gate, gamma, out
 * bf16). */
typedef struct {
  const void* y;
  int ldy;
  const void* gate;
  int ldg;
  const void* gamma;
  void* out;
  int ldo, rows, n;
  float eps;
} TfdGatedNormArgs;
int tfd_gated_rmsnorm_bf16(const TfdGatedNormArgs* args, void* stream);

/* Small-batch (1..4 sequences) C4 decode: a gated-DeltaNet layer in six launches
 * (the reference's tilelang runtime runs the mixer as three kernels,
 * examples/qwen3_5_35b_a3b-tilelang/kernels/gdn.py:1-60, and the MoE as router
 * logits, select and two expert kernels, kernels/moe.py:203-302, 368, 527).
 *
 * tfd_rowgemv_bf16: out[r][n] = bf16(sum_k W[n][k] x[r][k]) (TFD_EPI_LOGITS, f32
 * out) or out[r][n] += that (TFD_EPI_RESID_F32, in place) for r < rows <= 4, W
 * bf16 row-major [N][K], K 2048 or 4096, a wave per few rows (no MFMA padding).
 * The input rows x[r][0:K] are made by a prologue:
 *   TFD_ROWX_NORM_F32   f32 rows [rows][ldx] through RMSNorm with gamma [K], one
 *                       rounding (tfd_rmsnorm_f32_rows' arithmetic, bit for bit)
 *   TFD_ROWX_GATED_F32  Qwen3.5's gated output norm of the f32 read-out [rows][ldx]
 *                       per 128-value head with gate z f32 [rows][ldg] and gamma
 *                       [128]: bf16(x rsqrt(mean_head x^2 + eps) gamma silu(z))
 *                       (model.py:213-232; the sums of tfd_gdn_step)
 *   TFD_ROWX_OPERAND    bf16 rows in the skinny GEMMs' operand order
 *   TFD_ROWX_ROWS       bf16 rows [rows][ldx]
 * x_rows (optional): the prologue's bf16 rows [rows][ldxr] are also written there. */
#define TFD_ROWX_NORM_F32 0
#define TFD_ROWX_GATED_F32 1
#define TFD_ROWX_OPERAND 2
#define TFD_ROWX_ROWS 3
typedef struct {
  const void* x;
  int ldx, x_kind;
  const void* gamma;
  const float* gate;
  int ldg, head_dim;
  float eps;
  const void* w;
  int K, N;
  float* out;
  int ldo, epilogue;
  void* x_rows;
  int ldxr, rows;
} TfdRowGemvArgs;
int tfd_rowgemv_bf16(const TfdRowGemvArgs* args, void* stream);

/* tfd_gdn_step over value columns: blocks (value head, 32-column group, row),
 * 128 at batch 1.  The same inputs, state and window updates as tfd_gdn_step
 * (args->out and args->gamma are not used); the read-out before the gated
 * norm goes to read f32 [rows][ldr] (hv*128 values, bit-identical to the values
 * tfd_gdn_step normalises).  The gated norm is TFD_ROWX_GATED_F32 of the
 * out-projection. */
int tfd_gdn_step_cols(const TfdGdnArgs* args, float* read, int ldr, void* stream);

/* tfd_moe_experts for rows <= 4 in two launches: gate/up (each block routes its
 * row itself when route is TFD_MOE_ROUTE_SOFTMAX_TOPK, and writes weights / idx
 * as tfd_moe_experts does), then down + mix (+= into out with accumulate).  bf16
 * weights, TFD_POLICY_F32, hidden_size 2048, inter = shared_inter = 512, k <= 8;
 * groups and partial are not used.  Results equal tfd_moe_experts' bit for bit. */
int tfd_moe_experts_small(const TfdMoeArgs* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif
