/* C ABI of the MI355X (gfx950) decode-step library, libtfdecode_gfx950.so.
 *
 * Conventions for every entry:
 *   - pointers are device pointers (HBM) unless stated; sizes are plain ints;
 *   - `stream` is a hipStream_t passed as void*; work is enqueued on it and the
 *     entry returns without synchronising;
 *   - nothing is allocated: outputs and workspaces belong to the caller, so any
 *     sequence of calls can be captured in a HIP graph;
 *   - the return value is 0 on success, a negative code for a rejected argument
 *     (-1 bad pointer/argument, -2 bad shape, -3 unsupported size) or a positive
 *     hipError_t if the launch failed; tfd_last_error() gives the text;
 *   - values the kernels index memory with (token ids, positions, page-table
 *     entries) are checked on the device: a bad one sets a bit in `err`
 *     (TFD_ERR_*) and the access is skipped, never performed out of bounds.
 *
 * bf16 tensors are raw 16-bit bfloat16; weight matrices are row-major
 * [out][in].  The reference these entries replace is TileFoundry's Qwen3-1.7B
 * runtime, examples/qwen3_1_7b-tilelang/fast/kernels.py (tilelang kernels called
 * by fast/engine.py:189-217 and wrapped by fast/twin.py:112-226); the citation on
 * each entry names the reference kernel and the authored @func
 * (ref_src/model.py) whose semantics it computes.
 */
#ifndef TF_DECODE_H
#define TF_DECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TFD_ABI_VERSION 16

/* gemv prologues / epilogues */
#define TFD_PRO_PLAIN 0  /* x used as given */
#define TFD_PRO_NORM 1   /* x := Qwen3 RMSNorm(x) * gamma first */
#define TFD_EPI_STORE 0  /* out[n] = bf16(W[n].x) */
#define TFD_EPI_RESID 1  /* out[n] = bf16(resid[n] + bf16(W[n].x)) */
#define TFD_EPI_SWIGLU 2 /* rows are (gate_i, up_i) pairs: out[i] = bf16(bf16(silu(g)) * u) */
#define TFD_EPI_LOGITS 3 /* skinny GEMM only: out (f32) = bf16-valued W[n].x (the HIR's bf16 logits) */
#define TFD_EPI_RESID_F32 4 /* skinny GEMM only: out (f32) = resid (f32) + bf16-valued W[n].x; out may
                               be resid (an f32 residual stream, torch_ref.py:533-543) */

/* device error bits */
#define TFD_ERR_TOKEN_RANGE 1
#define TFD_ERR_POS_RANGE 2
#define TFD_ERR_PAGE_RANGE 4
#define TFD_ERR_STEP_RANGE 8

/* KV paging: a page holds 16 positions; a layer's pool is [pages][kv_heads][16][head_dim]
 * bf16 and position p of a sequence lives in page page_table[p / 16], row p % 16. */
#define TFD_PAGE_SIZE 16
/* context positions owned by one attention block */
#define TFD_ATTN_SPLIT 64

const char* tfd_last_error(void);
int tfd_abi_version(void);

/* out[i] = bf16(in[i]), round-to-nearest-even: the rounding every kernel applies
 * at the HIR's bf16 points (the evaluator's Tensor.to(bfloat16), ir/hir/tensor/cast.py:43). */
int tfd_round_bf16(const float* in, void* out, int n, void* stream);

/* RMSNorm with the Qwen3 rounding order: out = bf16(bf16(x*rsqrt(mean(x^2)+eps))*gamma).
 * Replaces fast/kernels.py:58-79 (rms_norm); semantics ref_src/model.py:125-137
 * (input_rms_norm) and :289-298 (final_rms_norm).  n % 8 == 0, n <= 8192. */
int tfd_rmsnorm_bf16(const void* x, const void* gamma, void* out, int n, float eps, void* stream);

/* out[0:hidden] = table[ids[0]].  Replaces fast/kernels.py:579-588 (embed);
 * semantics ref_src/model.py:279-287.  An id outside [0, vocab) sets TFD_ERR_TOKEN_RANGE. */
int tfd_embed_bf16(const void* table, const int64_t* ids, void* out, int hidden, int vocab,
                   int32_t* err, void* stream);

/* y = W x over N rows of length K, with an optional RMSNorm prologue and a fused
 * epilogue (TFD_PRO_*, TFD_EPI_*).  Replaces fast/kernels.py:123-145 (gemv),
 * :154-207 (gemv_attn_combine, minus the merge, which tfd_attn_pv_combine_paged
 * owns), :210-257 (gemv_silu) and :82-116 (resid_rms_norm, folded into the
 * prologue/epilogue); semantics ref_src/model.py:159-171, 213-215, 227-234, 264-266.
 * K % 8 == 0, K <= 8192; gamma only with TFD_PRO_NORM; resid only with TFD_EPI_RESID. */
int tfd_gemv_bf16(const void* x, const void* gamma, const void* w, const void* resid, void* out,
                  int K, int N, int prologue, int epilogue, float eps, void* stream);

/* Final norm, logits = bf16(W xn) for V rows (written as f32), and each of the
 * `nblocks` blocks' largest logit with the lowest index on ties.  Replaces
 * fast/kernels.py:260-321 (lm_head); semantics ref_src/model.py:300-305 and
 * generation.py:24-26.  block_val / block_idx hold nblocks entries. */
int tfd_lm_head_argmax_bf16(const void* x, const void* gamma, const void* w, float* logits,
                            float* block_val, int32_t* block_idx, int K, int V, int nblocks,
                            float eps, void* stream);

/* Greedy pick over the block partials (lowest index on ties); sam[pos] = pick;
 * ids[0] = inp[pos+1] while pos+1 < prompt_len, else the pick; pos += 1; and
 * hid = table[ids[0]] (the next step's embedding).  Replaces fast/kernels.py:591-637
 * (sample_step) plus the next step's embed. */
int tfd_argmax_finalize(const float* block_val, const int32_t* block_idx, int nblocks,
                        const int32_t* inp, const int32_t* prompt_len, int64_t* ids,
                        int32_t* pos, int32_t* sam, int nsteps, const void* table, void* hid,
                        int hidden, int vocab, int32_t* err, void* stream);

/* Attention part 1 over a paged cache.  From the bf16 [q | k | v] projection:
 * per-head q/k RMSNorm (gamma_q, gamma_k), RoPE at *rope_pos from the bf16 cos/sin
 * tables [rope_rows][head_dim], q_s = bf16(q_rope * scale); writes this token's
 * k_rope and v at position *cache_len of the cache; scores every prior position
 * j < *cache_len: scores[h][j] = bf16(sum_d bf16(q_s[h][d] * K[j][d])), the max per
 * TFD_ATTN_SPLIT split (split_max[nsplit][heads]) and the new key's score
 * (score_new[heads]).  Grid is nsplit x kv_heads; nsplit * 64 >= max_pages * 16.
 * Replaces fast/kernels.py:328-411 (qk_rope_cache) and the score half of :418-501
 * (attn_partial); semantics ref_src/model.py:172-198. */
int tfd_attn_rope_scores_paged(const void* qkv, const void* gamma_q, const void* gamma_k,
                               const void* cos_table, const void* sin_table, int rope_rows,
                               const int32_t* rope_pos, const int32_t* cache_len,
                               const int32_t* page_table, int max_pages, void* k_pool,
                               void* v_pool, int num_pages, int heads, int kv_heads,
                               int head_dim, float scale, float eps, float* scores,
                               int score_stride, float* split_max, float* score_new, int nsplit,
                               int32_t* err, void* stream);

/* Attention part 2: joint peak M, p_j = bf16(exp(bf16(s_j - M))), per-split sums of
 * p and bf16(p * V) in f32 (part_sum[nsplit][heads], part_out[nsplit][heads][head_dim]);
 * the last block per kv head (counted in counters[kv_heads], which must start at 0
 * and are left at 0) merges the splits with the new token's term:
 * attn = bf16(bf16(bf16(sum pV) + bf16(p_new v_new)) / bf16(bf16(sum p) + p_new)).
 * Replaces the softmax/PV half of fast/kernels.py:418-501 (attn_partial) and the
 * merge of :504-540 / :154-207; semantics ref_src/model.py:200-212. */
int tfd_attn_pv_combine_paged(const void* qkv, const int32_t* cache_len,
                              const int32_t* page_table, int max_pages, const void* v_pool,
                              int num_pages, int heads, int kv_heads, int head_dim,
                              const float* scores, int score_stride, const float* split_max,
                              const float* score_new, float* part_sum, float* part_out,
                              int nsplit, int32_t* counters, void* attn_out, int32_t* err,
                              void* stream);

/* ---- batched decode (workload C3: up to 32 sequences per step) -------
 * Row activations are row-major [rows][n] with leading dimensions; each sequence
 * has its own position (pos[b]) and page-table row (page_table + b * max_pages).
 * Activations that feed a skinny GEMM (normalised rows, attention output, SwiGLU
 * output) are kept in OPERAND ORDER instead: 32 rows x K bf16 where, for 32-wide k
 * step s and 16-row half h, the 1 KiB block at (2s + h) KiB holds at byte l * 16
 * X[16h + l % 16][32s + 8(l / 16) .. +7] (rows past the batch are never written).
 * This layout is internal to the batched path. */

/* Row-wise Qwen3 RMSNorm of `rows` vectors of n values (input_rms_norm per
 * sequence, ref_src/model.py:125-137).  n % 8 == 0, n <= 8192.  packed != 0: `out`
 * is in operand order (rows <= 32, n % 32 == 0; ldo unused). */
int tfd_rmsnorm_rows_bf16(const void* x, int ldx, const void* gamma, void* out, int ldo,
                          int rows, int n, float eps, int packed, void* stream);
/* The same norm written to both layouts in one launch: row-major out_rows
 * [rows][ldo] and/or out_packed in the skinny GEMMs' operand order (rows <= 32,
 * n % 32 == 0); NULL skips one. */
int tfd_rmsnorm_rows2_bf16(const void* x, int ldx, const void* gamma, void* out_rows, int ldo,
                           void* out_packed, int rows, int n, float eps, void* stream);

/* Weights [N][K] (row stride ldw) re-laid for tfd_gemm_skinny_bf16: 16-row x 32-k
 * blocks of 1 KiB in the matrix cores' operand order, rows padded with zeros to a
 * multiple of 16; `packed` holds ceil(N/16) * 16 * K bf16.  K % 256 == 0.  Done once
 * when a batched engine loads its weights.  The reference's kernels take weights as
 * ref_src/hf_alias.py:20-43 binds them ([in][out]); this layout is internal to the
 * batched path and has no counterpart there. */
int tfd_pack_skinny_bf16(const void* w, int ldw, int N, int K, void* packed, void* stream);

/* Skinny GEMM on the matrix cores: Y[m][n] = sum_k X[m][k] W[n][k] for m < M <= 32,
 * X in operand order (32 x K), W packed by tfd_pack_skinny_bf16 -- the q/k/v, o,
 * gate/up, down and head projections of a batch (ref_src/model.py:160-171, 213-215,
 * 230-234, 300-305 at M = batch; it replaces fast/kernels.py:123-145 / 260-321 at
 * batch > 1).  f32 accumulation, one rounding per output; epilogue TFD_EPI_STORE (out
 * [M][ldo]) / RESID (resid [M][ldr], out [M][ldo]) / SWIGLU (out [M][N/2] in operand
 * order, N/2 % 32 == 0; it feeds the down projection) / LOGITS (out f32 [M][ldo]).
 * K % 256 == 0.  Few-tile shapes (N/16 under four per compute unit, or K > 2048) split
 * K across the waves of a block and need no work buffer.  The others may split K
 * across blocks when `work` (work_floats f32 values, NULL with 0 allowed) permits: it
 * begins with TFD_SKINNY_COUNTERS int32 tile counters, zero before the first call
 * (every call leaves them at zero), followed by f32 partials of slices * ceil(N/16) *
 * 512 floats; the last wave to finish a tile adds its slices in slice order.  Calls
 * sharing one buffer must be stream-ordered. */
#define TFD_SKINNY_COUNTERS 16384
int tfd_gemm_skinny_bf16(const void* x, const void* w, int M, int K, int N, int epilogue,
                         const void* resid, int ldr, void* out, int ldo, float* work,
                         int64_t work_floats, void* stream);

/* tfd_gemm_skinny_bf16 that allocates nothing and takes no work buffer.  It has no
 * counterpart in the reference: it is for callers that cannot allocate (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  Its K-split
 * work (TFD_SKINNY_COUNTERS tile counters + 2^21 f32 partials, about 8 MiB) is a
 * device array inside the library, one per GPU, held until the process ends; the
 * first call on a device looks up its address.  The array is zero when the library
 * loads and every call leaves its counters at zero, so nothing is enqueued besides
 * the GEMM itself, also on a first call under stream capture.  The same
 * shapes and epilogues as tfd_gemm_skinny_bf16 (TFD_EPI_*), the results of that entry
 * with a work buffer of the same size (a K split across blocks is planned within the
 * scratch, with fewer slices where more would not fit).  Calls that overlap on one GPU
 * share the array and race: keep them stream-ordered. */
int tfd_gemm_skinny_bf16_noalloc(const void* x, const void* w, int M, int K, int N,
                                 int epilogue, const void* resid, int ldr, void* out, int ldo,
                                 void* stream);

/* tfd_attn_rope_scores_paged for `batch` sequences at once (grid nsplit x kv_heads x
 * batch): sequence b reads QKV row b (stride ldq) at its own position pos[b] and
 * page-table row b; its workspaces are the single-sequence ones at b * (their size).
 * Replaces fast/kernels.py:385-501 at batch > 1 (flash-decode over the paged cache). */
int tfd_attn_rope_scores_paged_batched(
    const void* qkv, int ldq, const void* gamma_q, const void* gamma_k, const void* cos_table,
    const void* sin_table, int rope_rows, const int32_t* pos, const int32_t* page_table,
    int max_pages, void* k_pool, void* v_pool, int num_pages, int batch, int heads, int kv_heads,
    int head_dim, float scale, float eps, float* scores, int score_stride, float* split_max,
    float* score_new, int nsplit, int split_tiles, int32_t* err, void* stream);

/* tfd_attn_pv_combine_paged for `batch` <= 32 sequences (counters: batch x kv_heads,
 * zero; the output rows go to attn_out in operand order, 32 x heads * head_dim, for
 * the o projection).  A split covers split_tiles x 64 positions in
 * both entries (long contexts: fewer, longer splits; one tile's loads are in flight
 * while the previous one is reduced); nsplit x split_tiles x 64 >= max_pages x 16.
 * split_tiles 0: each sequence's split length follows its position, ceil(ceil(pos /
 * 64) / nsplit) tiles, so its prior context spreads evenly over the nsplit splits at
 * every depth (score_stride >= max_pages x 16 rounded up to 64). */
int tfd_attn_pv_combine_paged_batched(
    const void* qkv, int ldq, const int32_t* pos, const int32_t* page_table, int max_pages,
    const void* v_pool, int num_pages, int batch, int heads, int kv_heads, int head_dim,
    const float* scores, int score_stride, const float* split_max, const float* score_new,
    float* part_sum, float* part_out, int nsplit, int split_tiles, int32_t* counters,
    void* attn_out, int32_t* err, void* stream);

/* Sampling a token per row of f32 logits (rows <= 65535, vocab <= TFD_SAMPLE_MAX_VOCAB),
 * on the device, in place of tfd_argmax_rows.  Replaces the reference's two samplers:
 *   top_k in 1..TFD_SAMPLE_MAX_K: the top k logits (ties to the lower index), divided by
 *     `temperature`, softmax over the k, the nucleus of mass `top_p` inside them (the
 *     tokens up to and including the one that crosses it, at least one), then one
 *     categorical draw (examples/qwen3_5_35b_a3b-tilelang/run.py:145-180);
 *   top_k = 0 (top_p must be 1): softmax(logits / temperature) over the whole row, by
 *     Gumbel-max (examples/granite_4_0_h_small-cuda/kernels/granite.cu:716-800).
 * The random numbers are a counter-based hash of (seed, row, counter[row], element):
 * pass each row's position (a device array the step advances) so that a captured graph
 * draws anew on every replay; NULL counts as 0.  NaN logits are never picked (an all-NaN
 * row picks 0).  `work`: tfd_sample_work_bytes(rows, vocab, top_k) bytes of device
 * memory, contents free.  Errors: kBadArg (null pointer, temperature <= 0, top_k out
 * of range, top_p outside (0, 1], or top_p < 1 with top_k = 0), kBadShape. */
#define TFD_SAMPLE_MAX_K 64
#define TFD_SAMPLE_MAX_VOCAB 262144
typedef struct TfdSampling {
  float temperature;
  int top_k;
  float top_p;
  uint64_t seed;
} TfdSampling;
int64_t tfd_sample_work_bytes(int rows, int vocab, int top_k);
int tfd_sample_rows(const float* logits, int ldl, int rows, int vocab,
                    const TfdSampling* sampling, const int32_t* counter, int32_t* pick,
                    void* work, int64_t work_bytes, void* stream);

/* Greedy pick per row: the first maximal logit (ref_src/generation.py:24-26).  With
 * `work` (rows * TFD_ARGMAX_WORK int32) the rows are scanned by 64 blocks each and the
 * chunk winners reduced by a second launch; NULL scans each row with one block. */
#define TFD_ARGMAX_WORK 128
int tfd_argmax_rows(const float* logits, int ldl, int rows, int vocab, int32_t* pick,
                    int32_t* work, void* stream);

/* The step's last node per sequence (the batch form of tfd_argmax_finalize,
 * fast/kernels.py:591-637): record pick[b] at sam[b][pos[b]], feed the next prompt
 * token while sequence b's prompt lasts and the pick after, advance pos[b], stage the
 * next token's embedding row in hid row b. */
int tfd_finalize_rows(const int32_t* pick, int rows, const int32_t* inp, int ld_inp,
                      const int32_t* prompt_len, int64_t* ids, int32_t* pos, int32_t* sam,
                      int ld_sam, int nsteps, const void* table, void* hid, int ldh, int hidden,
                      int vocab, int32_t* err, void* stream);

/* Embedding rows of ids[0..rows) (Qwen3_1_7B.embed per sequence, ref_src/model.py:279-287). */
int tfd_embed_rows_bf16(const void* table, const int64_t* ids, void* out, int ldo, int rows,
                        int hidden, int vocab, int32_t* err, void* stream);

/* ---- persistent decode step ------------------------------------------------
 * One cooperative launch runs `steps` whole decode steps (every layer, the head,
 * the greedy pick, the next embedding), instead of ~6 launches per layer.  No
 * grid barrier: every block polls for the data it needs (flag-in-data words),
 * so a phase starts in each block as soon as its inputs exist.  It computes
 * exactly what the per-kernel entries above compute, with the same arithmetic
 * in the same order, so the two paths give identical bits.
 * Replaces the captured step of fast/engine.py:189-217 (graph.replay per token). */
typedef struct TfdLayer {
  const void* w_qkv;      /* [HQ*D + 2*HKV*D][H] bf16: q rows, k rows, v rows */
  const void* w_o;        /* [H][HQ*D] */
  const void* w_gu;       /* [2*I][H], gate_i at row 2i and up_i at row 2i+1 */
  const void* w_down;     /* [H][I] */
  const void* gamma_in;   /* [H] */
  const void* gamma_post; /* [H] */
  const void* gamma_q;    /* [D] */
  const void* gamma_k;    /* [D] */
  void* k_pool;           /* [num_pages][HKV][16][D] */
  void* v_pool;
} TfdLayer;

typedef struct TfdDecodeArgs {
  const TfdLayer* layers; /* device array of n_layers entries */
  int n_layers, hidden, heads, kv_heads, head_dim, intermediate, vocab;
  float eps, scale;       /* rms eps; the bf16 value of head_dim^-0.5 */
  const void* w_embed;    /* [V][H] */
  const void* w_head;     /* [V][H] (the embedding table when tied) */
  const void* gamma_final;
  const void* cos_table;  /* [rope_rows][D] bf16 */
  const void* sin_table;
  int rope_rows;
  const int32_t* page_table;
  int max_pages, num_pages;
  /* Blocks exchange data through flag-in-data words: 8 bytes, a 32-bit payload
   * (a bf16 pair or an f32) and the 32-bit tag of the step and layer that wrote
   * it.  Zero these buffers once when they are allocated; tags then continue
   * across launches from `epoch`, which the caller advances by
   * TFD_TAGS_PER_STEP(n_layers) for every step run (and, before it would pass
   * 2^32, zeroes the buffers again and restarts at 0). */
  uint32_t* x_hid;        /* [H/2] words: the hidden state entering a layer or the head */
  uint32_t* x_h1;         /* [H/2]: after attention and its residual */
  uint32_t* x_qkv;        /* [(HQ*D + 2*HKV*D)/2] */
  uint32_t* x_attn;       /* [HQ*D/2] */
  uint32_t* x_mid;        /* [I/2] */
  uint32_t* x_smax;       /* [nsplit][HQ] */
  uint32_t* x_psum;       /* [nsplit][HQ] */
  uint32_t* x_pout;       /* [nsplit][HQ][D] */
  uint32_t* x_best;       /* [2 x grid blocks] */
  uint32_t epoch;
  float* scores;          /* [HQ][score_stride] workspace */
  int score_stride;
  float* score_new;       /* [HQ] workspace */
  int nsplit;             /* >= ceil(max position + 1, 64) */
  float* logits;          /* [V], the last step's */
  int64_t* ids;           /* the token entering the next step */
  int32_t* pos;           /* its position */
  const int32_t* inp;     /* [nsteps] prompt ids */
  const int32_t* prompt_len;
  int32_t* sam;           /* [nsteps] picks */
  int nsteps;
  int32_t* err;
  /* Optional phase timeline (may be null): for the first timeline_steps steps of
   * a launch, every block records the 100 MHz device wall clock when each
   * phase's input is ready and when its output is out: [step][block][stamp],
   * TFD_TIMELINE_STAMPS(n_layers) stamps per step and block. */
  uint64_t* timeline;
  int timeline_steps;
} TfdDecodeArgs;

/* per layer 7 phases (qkv, scores, P.V, merge, o, gate/up, down), then head and pick */
#define TFD_TIMELINE_STAMPS(n_layers) (14 * (n_layers) + 4)
#define TFD_TAGS_PER_STEP(n_layers) ((n_layers) + 1)

#define TFD_ERR_SYNC 16 /* a wait for another block's data passed its bound; the launch gave up */
#define TFD_ERR_PLACEMENT 32 /* tfd_decode_xcd: a block read an XCC id outside 0..7 */

/* Run `steps` decode steps in one launch.  nblocks <= 0 picks one block per
 * compute unit.  Returns -3 if the shape has no persistent instance (hidden
 * must equal heads * head_dim) or the grid cannot be co-resident. */
int tfd_decode_persistent(const TfdDecodeArgs* args, int steps, int nblocks, void* stream);
/* The grid tfd_decode_persistent(args, ., 0, .) uses (x_best must hold 2x this many words). */
int tfd_decode_persistent_grid(void);

/* The exchange buffers of tfd_decode_xcd beyond those of TfdDecodeArgs (flag-in-data
 * words as there; zero once, tags from args->epoch).  Per XCD x of the 8: */
typedef struct TfdXcdArgs {
  uint32_t* hid;   /* [8][H/2]: the hidden state entering a layer, XCD x's copy at x * H/2 */
  uint32_t* h1;    /* [8][H/2]: after attention and its residual */
  uint32_t* opart; /* [8][H]: XCD x's partial o-projection sums (f32) */
  uint32_t* dpart; /* [8][H]: XCD x's partial down-projection sums (f32) */
  uint32_t* smax;  /* [8][nsplit][HQ]: XCD x's split maxima */
  uint32_t* psum;  /* [8][nsplit][HQ] */
  uint32_t* pout;  /* [8][nsplit][HQ][D] */
} TfdXcdArgs;

/* tfd_decode_persistent with the layer split over the device's 8 XCDs (256 compute
 * units: 32 per XCD) so that most hand-offs stay inside one XCD's L2: XCD x holds
 * kv head x, its query heads, 1/8 of the SwiGLU columns and the matching K slices
 * of o and down, whose products are summed over XCDs by an all-reduce (two per
 * layer).  Same step as tfd_decode_persistent (examples/qwen3_1_7b-tilelang/fast/
 * engine.py:189-217); the o and down sums add their XCD slices in a different f32
 * order.  For the Qwen3-1.7B shape only (hidden 2048, 16 q / 8 kv heads of 128,
 * intermediate 6144); -3 otherwise or on a device that is not 8 x 32 compute units.
 * args->x_hid, x_h1, x_smax, x_psum and x_pout are not used (the XCD arenas replace
 * them); nsplit <= 128.  Block b plays the XCD of its hardware XCC id as rank b / 8;
 * an XCC id outside 0..7 raises TFD_ERR_PLACEMENT | TFD_ERR_SYNC and the launch gives
 * up, and a placement that is not round-robin over the XCDs leaves some rank unplayed,
 * which ends the launch with TFD_ERR_SYNC. */
int tfd_decode_xcd(const TfdDecodeArgs* args, const TfdXcdArgs* xcd, int steps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TF_DECODE_H */
