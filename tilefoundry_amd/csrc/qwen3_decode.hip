// Qwen3 dense decode step, batch 1, bf16, for gfx950.
//
// One library, exported through the C ABI declared in include/tf_decode.h.
// Every entry takes raw device pointers, plain integer sizes and a hipStream_t,
// allocates nothing and never synchronises, so a caller may capture any
// sequence of them in a graph.  Outputs and workspaces are caller-owned.
//
// Kernels of one layer (the reference's fast/kernels.py does the same work in
// eight tilelang kernels; this file folds it into six):
//   gemv<NORM, STORE>   rmsnorm(x) @ [q|k|v]^T            -> qkv (bf16)
//   attn_rope_scores    q/k RMS + RoPE, K/V page write, q.K -> scores, split max
//   attn_pv_combine     softmax numerators, P.V per split, last block merges
//   gemv<PLAIN, RESID>  attn @ Wo^T + residual             -> h1
//   gemv<NORM, SWIGLU>  rmsnorm(h1) @ [gate,up]^T, silu*up -> h (intermediate)
//   gemv<PLAIN, RESID>  h @ Wdown^T + residual             -> next hidden
// and per step: lm_head_argmax (final norm, logits, block argmax) and
// argmax_finalize (global argmax, next token, position, next embedding row).
//
// Weights are row-major [out][in] bf16, so a row is one contiguous dot product
// and the tied head reads the embedding table in place.

#include "decode_phases.h"
#include "host_common.h"
#include "tf_decode.h"

#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

using namespace tfd;
using namespace tfd_host;

namespace {

constexpr float kNegInfHost = -__builtin_huge_valf();

// ---------------------------------------------------------------------------
// Standalone RMSNorm (input_rms_norm / final_rms_norm, model.py:125-137, 289-298)
// ---------------------------------------------------------------------------
template <int kCmax>
__global__ __launch_bounds__(kWave) void k_rmsnorm(const bf16* __restrict__ x,
                                                   const bf16* __restrict__ gamma,
                                                   bf16* __restrict__ out, int n, float eps) {
  const int lane = threadIdx.x;
  u32x4 xr[kCmax];
  rms_norm_x<kCmax>(x, gamma, n, eps, lane, xr);
  const int nch = n / 8;
#pragma unroll
  for (int i = 0; i < kCmax; ++i) {
    const int c = i * kWave + lane;
    if (c < nch) *reinterpret_cast<u32x4*>(out + (int64_t)c * 8) = xr[i];
  }
}

// ---------------------------------------------------------------------------
// Embedding row gather (model.py:279-287)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void k_round_bf16(const float* __restrict__ in,
                                                       bf16* __restrict__ out, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = f2bf(in[i]);
}

__global__ __launch_bounds__(kBlock) void k_embed(const bf16* __restrict__ table,
                                                  const int64_t* __restrict__ ids,
                                                  bf16* __restrict__ out, int hidden, int vocab,
                                                  int* err) {
  int64_t id = ids[0];
  if (id < 0 || id >= vocab) {
    if (threadIdx.x == 0 && blockIdx.x == 0) raise_error(err, kErrTokenRange);
    id = 0;
  }
  const bf16* row = table + id * (int64_t)hidden;
  for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < hidden / 8;
       c += gridDim.x * blockDim.x)
    *reinterpret_cast<u32x4*>(out + (int64_t)c * 8) = load16(row + (int64_t)c * 8);
}


// ---------------------------------------------------------------------------
// one kernel per phase (virtual block = blockIdx)
// ---------------------------------------------------------------------------
template <int kCmax, int kR, int kPro, int kEpi>
__global__ __launch_bounds__(kBlock) void k_gemv(const bf16* __restrict__ x,
                                                 const bf16* __restrict__ gamma,
                                                 const bf16* __restrict__ W,
                                                 const bf16* __restrict__ resid,
                                                 bf16* __restrict__ out, int K, int N, float eps) {
  gemv_phase<kCmax, kR, kPro, kEpi>(blockIdx.x, x, gamma, W, resid, out, K, N, eps);
}

template <int kCmax, int kR>
__global__ __launch_bounds__(kBlock) void k_lm_head_argmax(
    const bf16* __restrict__ x, const bf16* __restrict__ gamma, const bf16* __restrict__ W,
    float* __restrict__ logits, float* __restrict__ bv, int* __restrict__ bi, int K, int V,
    float eps) {
  lm_head_phase<kCmax, kR>(blockIdx.x, gridDim.x, x, gamma, W, logits, bv, bi, K, V, eps);
}

__global__ __launch_bounds__(1024) void k_argmax_finalize(
    const float* __restrict__ bv, const int* __restrict__ bi, int nb,
    const int* __restrict__ inp, const int* __restrict__ plen, int64_t* __restrict__ ids,
    int* __restrict__ pos, int* __restrict__ sam, int nsteps, const bf16* __restrict__ table,
    bf16* __restrict__ hid, int hidden, int vocab, int* err) {
  finalize_phase(bv, bi, nb, inp, plen, ids, pos, sam, nsteps, table, hid, hidden, vocab, err);
}

template <int D, int G>
__global__ __launch_bounds__(kBlock) void k_attn_rope_scores(
    const bf16* __restrict__ qkv, const bf16* __restrict__ gq, const bf16* __restrict__ gk,
    const bf16* __restrict__ cos_t, const bf16* __restrict__ sin_t, int rope_rows,
    const int* __restrict__ rope_pos, const int* __restrict__ cache_len,
    const int* __restrict__ page_table, int max_pages, bf16* __restrict__ kpool,
    bf16* __restrict__ vpool, int num_pages, int kv_heads, float scale, float eps,
    float* __restrict__ S, int s_stride, float* __restrict__ smax, float* __restrict__ snew,
    int* err) {
  const int P = coh_ldi(cache_len);
  KTile<D> kt;
  k_tile_issue<D, false>(blockIdx.x, blockIdx.y, P, page_table, max_pages, kpool, num_pages, kv_heads,
                  kt);
  const int rp = coh_ldi(rope_pos);
  const QKPre pre = qk_prefetch<D, G>(rp, P, gq, gk, cos_t, sin_t, rope_rows, page_table,
                                      max_pages);
  __shared__ __attribute__((aligned(16))) uint32_t hs[(G + 2) * D / 2];
  stage_head<D, G>(blockIdx.y, kv_heads * G, kv_heads, qkv, hs);
  __syncthreads();
  attn_scores_phase<D, G, false>(blockIdx.x, blockIdx.y, hs, pre, rope_rows, rp, P, page_table,
                                 max_pages, kpool, vpool, num_pages, kv_heads, scale, eps, S,
                                 s_stride, smax, snew, AttnLL{}, kt, err);
}

template <int D, int G>
__global__ __launch_bounds__(kBlock) void k_attn_pv_combine(
    const bf16* __restrict__ qkv, const int* __restrict__ cache_len,
    const int* __restrict__ page_table, int max_pages, const bf16* __restrict__ vpool,
    int num_pages, int kv_heads, const float* __restrict__ S, int s_stride,
    const float* __restrict__ smax, const float* __restrict__ snew, float* part_sum,
    float* part_out, int* counters, bf16* __restrict__ attn_out, int* err) {
  int P = coh_ldi(cache_len);
  if (P < 0 || P >= max_pages * kPage) P = 0;
  VTile<D> vt;
  v_tile_issue<D, false>(blockIdx.x, blockIdx.y, P, page_table, max_pages, vpool, num_pages, kv_heads,
                  vt);
  attn_pv_phase<D, G, false>(blockIdx.x, blockIdx.y, gridDim.x, qkv, P, page_table, max_pages,
                             vpool, num_pages, kv_heads, S, s_stride, smax, snew, part_sum,
                             part_out, counters, attn_out, AttnLL{}, vt, err);
}

// ---------------------------------------------------------------------------
// lm_head for the persistent kernel: the same per-row arithmetic as
// lm_head_phase, with the block's row groups double-buffered in registers so
// the next group's loads are in flight while the current one is reduced.
// ---------------------------------------------------------------------------
template <int kCmax, int kR>
__device__ __forceinline__ void lm_head_rows(int64_t row0, int V, int lane,
                                             const u32x4 (&xr)[kCmax],
                                             const u32x4 (&w)[kR][kCmax], float* logits,
                                             float& best, int& besti) {
  if (row0 >= V) return;
  const int nvalid = (int)((V - row0) < kR ? (V - row0) : kR);
  float acc[kR];
  dot_loaded<kCmax, kR>(w, xr, acc);
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    if (r < nvalid) {
      const float y = rbf(acc[r]);
      if (lane == r) logits[row0 + r] = y;
      if (better(y, (int)(row0 + r), best, besti)) {
        best = y;
        besti = (int)(row0 + r);
      }
    }
  }
}

// xr: the normalised final hidden state.  Publishes the block's pick as a
// flag-in-data (value, index) pair.
template <int kCmax, int kR>
__device__ __forceinline__ void lm_head_ll(const u32x4 (&xr)[kCmax], const bf16* __restrict__ W,
                                           float* logits, uint32_t* best_ll, uint32_t tag, int K,
                                           int V, u32x4 (&wa)[kR][kCmax]) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock * kR;
  int64_t r0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * kR;
  u32x4 wb[kR][kCmax];
  float best = kNegInf;
  int besti = 0x7fffffff;
  while (r0 < V) {
    const int64_t r1 = r0 + stride;
    gemv_issue<kCmax, kR>((int)(r1 / (kWavesPerBlock * kR)), W, K, V, wb);
    lm_head_rows<kCmax, kR>(r0, V, lane, xr, wa, logits, best, besti);
    if (r1 >= V) break;
    const int64_t r2 = r1 + stride;
    gemv_issue<kCmax, kR>((int)(r2 / (kWavesPerBlock * kR)), W, K, V, wa);
    lm_head_rows<kCmax, kR>(r1, V, lane, xr, wb, logits, best, besti);
    r0 = r2;
  }
  __shared__ float sv[kWavesPerBlock];
  __shared__ int si[kWavesPerBlock];
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = besti;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int i = si[0];
    for (int w = 1; w < kWavesPerBlock; ++w)
      if (better(sv[w], si[w], b, i)) {
        b = sv[w];
        i = si[w];
      }
    ll_put2(best_ll, 2u * blockIdx.x, __float_as_uint(b), (uint32_t)i, tag);
  }
  __syncthreads();
}

__device__ __forceinline__ void stamp(uint64_t*& tl) {
  if (tl && threadIdx.x == 0) *tl++ = wall_clock64();
}

// ---------------------------------------------------------------------------
// The persistent decode kernel: `steps` whole decode steps in one launch, with
// no grid barrier.  Blocks hand data to each other as flag-in-data words tagged
// with the (step, layer), and each block polls for exactly what it needs:
//   qkv    x = the hidden state (the embedding row at layer 0, which every block
//          reads from the table itself) -> QKV
//   attn   head slices of QKV -> scores, split maxima -> P.V partials ->
//          merged output (part 1, 2, 3; each block runs all its part-1 work
//          before it waits in part 2, and all its part-2 work before part 3,
//          so no wait can depend on work queued behind it)
//   o      x = attention output, residual = the hidden state kept in LDS -> h1
//   gu     x = h1 (kept in LDS for the down residual) -> SwiGLU output
//   down   x = SwiGLU output -> the next hidden state
//   head   x = the last hidden state -> logits and one (value, index) per block;
//          every block reduces all of them and knows the next token.
// The next phase's weights are issued before the wait for its input, so HBM
// streams while the data arrives.  Row tiles are sized so each GEMV phase is one
// round of loads per wave on a 256-block grid at the Qwen3-1.7B shape (qkv
// 4096 = 1024 waves x 4 rows, o 2048 x 2, gate/up 12288 x 12, down 2048 x 2);
// other shapes loop.
// ---------------------------------------------------------------------------
template <int kCH, int kCI, int D, int G>
__global__ __launch_bounds__(kBlock) void k_decode_persistent(TfdDecodeArgs a, int steps) {
  constexpr int kRqkv = 4, kRo = 2, kRgu = 12, kRdown = 2, kRhead = 4;
  constexpr int kXs = (kCH > kCI ? kCH : kCI) * kWave * 4;   // words: the longest x
  __shared__ __attribute__((aligned(16))) uint32_t xs[kXs];
  __shared__ __attribute__((aligned(16))) uint32_t hid_s[kCH * kWave * 4];
  __shared__ __attribute__((aligned(16))) uint32_t h1_s[kCH * kWave * 4];
  __shared__ __attribute__((aligned(16))) uint32_t hs[(G + 2) * D / 2];
  // each attention work item's scores and new-key scores stay in LDS from part
  // 1 to parts 2 and 3 (a block runs at most kMaxItems items per layer)
  constexpr int kMaxItems = 4;
  __shared__ float s_sc[kMaxItems][G * kSplit];
  __shared__ float s_new[kMaxItems][G];
  const int nb = gridDim.x;
  const int H = a.hidden, I = a.intermediate, V = a.vocab;
  const int QD = a.heads * D;
  const int qkv_n = QD + 2 * a.kv_heads * D;
  const float eps = a.eps;
  const int vb0 = blockIdx.x;
  int* const err = a.err;
  int P = coh_ldi(a.pos);   // position of this step; advances by one per step
  int tok = (int)__hip_atomic_load(a.ids, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  const int lane = threadIdx.x & (kWave - 1);
  u32x4 wq[kRqkv][kCH], wo[kRo][kCH], wg[kRgu][kCH], wd[kRdown][kCI];
  u32x4 gq_in[kCH], gq_post[kCH];   // norm scales, prefetched with the weights
  gemv_issue<kCH, kRqkv>(vb0, (const bf16*)a.layers[0].w_qkv, H, qkv_n, wq);
  load_x<kCH>((const bf16*)a.layers[0].gamma_in, H / 8, lane, gq_in);
  for (int t = 0; t < steps; ++t, ++P) {
    uint64_t* tl = (a.timeline && t < a.timeline_steps)
                       ? a.timeline + ((int64_t)t * nb + blockIdx.x) * (14 * a.n_layers + 4)
                       : nullptr;
    const uint32_t tag0 = a.epoch + (uint32_t)t * (uint32_t)(a.n_layers + 1);
    // this step's input: the embedding row of the current token
    {
      const int id = (tok >= 0 && tok < V) ? tok : 0;
      const uint32_t* row = reinterpret_cast<const uint32_t*>((const bf16*)a.w_embed +
                                                              (int64_t)id * H);
      for (int i = threadIdx.x; i < H / 8; i += kBlock)
        *reinterpret_cast<u32x4*>(hid_s + 4 * i) = *reinterpret_cast<const u32x4*>(row + 4 * i);
    }
    // attention shape at this position (an out-of-range position has raised
    // its error in part 1; the shape then stays that of position 0)
    const int Pc = (P >= 0 && P < a.max_pages * kPage) ? P : 0;
    const int nact = (Pc + kSplit - 1) / kSplit;
    const int parts = nact > 0 ? nact : 1;
    const int nvb = parts * a.kv_heads;
    for (int l = 0; l < a.n_layers; ++l) {
      const TfdLayer w = a.layers[l];
      const uint32_t tag = tag0 + (uint32_t)l + 1u;
      // ---- qkv
      if (l > 0) ll_stage(a.x_hid, H, tag - 1u, hid_s, err);
      __syncthreads();
      stamp(tl);
      gemv_ll<kCH, kRqkv, kNorm, kStore>(hid_s, gq_in, (const bf16*)w.w_qkv, nullptr, a.x_qkv,
                                         tag, H, qkv_n, eps, wq);
      stamp(tl);
      // the o projection's weights and this block's first K / V tiles stream
      // while the QKV projection arrives
      gemv_issue<kCH, kRo>(vb0, (const bf16*)w.w_o, QD, H, wo);
      KTile<D> kt;
      VTile<D> vt;
      const int s0 = vb0 < nvb ? vb0 % parts : parts, h0 = vb0 / parts;
      k_tile_issue<D, true>(s0, h0, P, a.page_table, a.max_pages, (const bf16*)w.k_pool, a.num_pages,
                      a.kv_heads, kt);
      v_tile_issue<D, true>(s0, h0, P, a.page_table, a.max_pages, (const bf16*)w.v_pool, a.num_pages,
                      a.kv_heads, vt);
      const QKPre pre = qk_prefetch<D, G>(P, P, (const bf16*)w.gamma_q, (const bf16*)w.gamma_k,
                                          (const bf16*)a.cos_table, (const bf16*)a.sin_table,
                                          a.rope_rows, a.page_table, a.max_pages);
      const AttnLL ll{a.x_qkv, a.x_smax, a.x_psum, a.x_pout, a.x_attn, tag};
      // ---- attention part 1: scores
      for (int vb = vb0; vb < nvb; vb += nb) {
        const int split = vb % parts, h = vb / parts;
        if (vb != vb0)
          k_tile_issue<D, true>(split, h, P, a.page_table, a.max_pages, (const bf16*)w.k_pool,
                          a.num_pages, a.kv_heads, kt);
        stage_head_ll<D, G>(h, a.heads, a.kv_heads, ll, hs, err);
        __syncthreads();
        if (vb == vb0) stamp(tl);
        const int lv = (vb - vb0) / nb;
        attn_scores_phase<D, G, true>(split, h, hs, pre, a.rope_rows, P, P, a.page_table,
                                      a.max_pages, (bf16*)w.k_pool, (bf16*)w.v_pool,
                                      a.num_pages, a.kv_heads, a.scale, eps, s_sc[lv], 0,
                                      nullptr, s_new[lv], ll, kt, err);
        if (vb == vb0) stamp(tl);
      }
      // ---- part 2: P.V partials
      for (int vb = vb0; vb < nvb; vb += nb) {
        const int split = vb % parts, h = vb / parts;
        if (vb != vb0)
          v_tile_issue<D, true>(split, h, P, a.page_table, a.max_pages, (const bf16*)w.v_pool,
                          a.num_pages, a.kv_heads, vt);
        if (vb == vb0) stamp(tl);
        const int lv = (vb - vb0) / nb;
        attn_pv_phase<D, G, true>(split, h, a.nsplit, nullptr, P, a.page_table, a.max_pages,
                                  (const bf16*)w.v_pool, a.num_pages, a.kv_heads, s_sc[lv], 0,
                                  nullptr, s_new[lv], nullptr, nullptr, nullptr, nullptr, ll, vt,
                                  err);
        if (vb == vb0) stamp(tl);
      }
      // ---- part 3: merge
      for (int vb = vb0; vb < nvb; vb += nb) {
        if (vb == vb0) stamp(tl);
        attn_merge_ll<D, G>(vb % parts, vb / parts, P, a.max_pages, a.kv_heads,
                            s_new[(vb - vb0) / nb], ll, err);
        __syncthreads();
        if (vb == vb0) stamp(tl);
      }
      if (vb0 >= nvb) {
        stamp(tl); stamp(tl); stamp(tl); stamp(tl); stamp(tl); stamp(tl);
      }
      // ---- o projection + residual
      ll_stage(a.x_attn, QD, tag, xs, err);
      __syncthreads();
      stamp(tl);
      // (a plain prologue takes no norm scales: any array of the right shape will do)
      gemv_ll<kCH, kRo, kPlain, kResid>(xs, gq_post, (const bf16*)w.w_o, hid_s, a.x_h1, tag, QD,
                                        H, eps, wo);
      stamp(tl);
      gemv_issue<kCH, kRgu>(vb0, (const bf16*)w.w_gu, H, 2 * I, wg);
      load_x<kCH>((const bf16*)w.gamma_post, H / 8, lane, gq_post);
      // ---- gate/up + SwiGLU
      ll_stage(a.x_h1, H, tag, h1_s, err);
      __syncthreads();
      stamp(tl);
      gemv_ll<kCH, kRgu, kNorm, kSwiglu>(h1_s, gq_post, (const bf16*)w.w_gu, nullptr, a.x_mid,
                                         tag, H, 2 * I, eps, wg);
      stamp(tl);
      gemv_issue<kCI, kRdown>(vb0, (const bf16*)w.w_down, I, H, wd);
      // ---- down + residual
      ll_stage(a.x_mid, I, tag, xs, err);
      __syncthreads();
      stamp(tl);
      gemv_ll<kCI, kRdown, kPlain, kResid>(xs, wd[0], (const bf16*)w.w_down, h1_s, a.x_hid, tag,
                                           I, H, eps, wd);
      stamp(tl);
      // the next layer's qkv weights -- or, after the last layer, layer 0's for
      // the next step (issued unconditionally: a conditional issue would keep
      // the tile live through the whole step); the head streams its own
      gemv_issue<kCH, kRqkv>(vb0, (const bf16*)a.layers[(l + 1) % a.n_layers].w_qkv, H, qkv_n,
                             wq);
      load_x<kCH>((const bf16*)a.layers[(l + 1) % a.n_layers].gamma_in, H / 8, lane, gq_in);
      __syncthreads();
    }
    // ---- head: final norm, logits, block pick
    {
      const uint32_t tag_head = tag0 + (uint32_t)a.n_layers;
      u32x4 wa[kRhead][kCH], gr[kCH];
      gemv_issue<kCH, kRhead>(vb0, (const bf16*)a.w_head, H, V, wa);
      load_x<kCH>((const bf16*)a.gamma_final, H / 8, lane, gr);
      ll_stage(a.x_hid, H, tag_head, hid_s, err);
      __syncthreads();
      stamp(tl);
      u32x4 xr[kCH];
      x_from_lds<kCH>(hid_s, H / 8, lane, xr);
      rms_norm_apply<kCH>(xr, gr, H, eps);
      lm_head_ll<kCH, kRhead>(xr, (const bf16*)a.w_head, a.logits, a.x_best, tag_head + 1u, H, V,
                              wa);
      stamp(tl);
    }
    // ---- the pick and the next token (every block)
    stamp(tl);
    tok = finalize_ll(a.x_best, nb, tag0 + (uint32_t)a.n_layers + 1u, P, a.inp, a.prompt_len,
                      a.nsteps, V, a.ids, a.pos, a.sam, err);
    stamp(tl);
    if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSync) break;
  }
}

// ---------------------------------------------------------------------------
// host side: argument checks, error text, launches
// ---------------------------------------------------------------------------
template <int kC, int kR, int kPro, int kEpi>
void launch_gemv(const bf16* x, const bf16* gamma, const bf16* W, const bf16* resid, bf16* out,
                 int K, int N, float eps, hipStream_t s) {
  const int rows_per_block = kWavesPerBlock * kR;
  const int grid = (N + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((k_gemv<kC, kR, kPro, kEpi>), dim3(grid), dim3(kBlock), 0, s, x, gamma, W,
                     resid, out, K, N, eps);
}

}  // namespace


namespace tfd_host {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

int compute_units() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

int cmax_for(int K) {
  const int per_lane = (K / 8 + kWave - 1) / kWave;
  if (per_lane <= 1) return 1;
  if (per_lane <= 2) return 2;
  if (per_lane <= 4) return 4;
  if (per_lane <= 8) return 8;
  if (per_lane <= 12) return 12;
  if (per_lane <= 16) return 16;
  return 0;
}

}  // namespace tfd_host

extern "C" {

const char* tfd_last_error(void) { return tfd_host::g_err; }

int tfd_abi_version(void) { return TFD_ABI_VERSION; }

int tfd_rmsnorm_bf16(const void* x, const void* gamma, void* out, int n, float eps,
                     void* stream) {
  if (!x || !gamma || !out) return fail(kBadArg, "rmsnorm: null pointer");
  if (n <= 0 || n % 8) return fail(kBadShape, "rmsnorm: n=%d must be a positive multiple of 8", n);
  auto s = (hipStream_t)stream;
  TFD_CMAX_SWITCH(n, hipLaunchKernelGGL((k_rmsnorm<kC>), dim3(1), dim3(kWave), 0, s,
                                        (const bf16*)x, (const bf16*)gamma, (bf16*)out, n, eps));
  return launched("rmsnorm");
}

int tfd_round_bf16(const float* in, void* out, int n, void* stream) {
  if (!in || !out) return fail(kBadArg, "round_bf16: null pointer");
  if (n <= 0) return fail(kBadShape, "round_bf16: n=%d", n);
  const int grid = (n + kBlock - 1) / kBlock < 1024 ? (n + kBlock - 1) / kBlock : 1024;
  hipLaunchKernelGGL(k_round_bf16, dim3(grid), dim3(kBlock), 0, (hipStream_t)stream, in,
                     (bf16*)out, n);
  return launched("round_bf16");
}

int tfd_embed_bf16(const void* table, const int64_t* ids, void* out, int hidden, int vocab,
                   int32_t* err, void* stream) {
  if (!table || !ids || !out) return fail(kBadArg, "embed: null pointer");
  if (hidden <= 0 || hidden % 8 || vocab <= 0)
    return fail(kBadShape, "embed: hidden=%d (multiple of 8), vocab=%d", hidden, vocab);
  const int grid = (hidden / 8 + kBlock - 1) / kBlock;
  hipLaunchKernelGGL(k_embed, dim3(grid), dim3(kBlock), 0, (hipStream_t)stream,
                     (const bf16*)table, ids, (bf16*)out, hidden, vocab, err);
  return launched("embed");
}

int tfd_gemv_bf16(const void* x, const void* gamma, const void* w, const void* resid, void* out,
                  int K, int N, int prologue, int epilogue, float eps, void* stream) {
  if (!x || !w || !out) return fail(kBadArg, "gemv: null pointer");
  if (prologue == TFD_PRO_NORM && !gamma) return fail(kBadArg, "gemv: norm prologue needs gamma");
  if (epilogue == TFD_EPI_RESID && !resid) return fail(kBadArg, "gemv: residual epilogue needs resid");
  if (K <= 0 || K % 8 || N <= 0) return fail(kBadShape, "gemv: K=%d (multiple of 8), N=%d", K, N);
  if (epilogue == TFD_EPI_SWIGLU && N % 2)
    return fail(kBadShape, "gemv: swiglu epilogue needs an even row count, N=%d", N);
  auto s = (hipStream_t)stream;
  auto xb = (const bf16*)x;
  auto gb = (const bf16*)gamma;
  auto wb = (const bf16*)w;
  auto rb = (const bf16*)resid;
  auto ob = (bf16*)out;
  const bool norm = prologue == TFD_PRO_NORM;
  if (prologue != TFD_PRO_PLAIN && prologue != TFD_PRO_NORM)
    return fail(kBadArg, "gemv: prologue %d", prologue);
  switch (epilogue) {
    case TFD_EPI_STORE:
      if (norm) {
        TFD_CMAX_SWITCH(K, (launch_gemv<kC, 4, kNorm, kStore>(xb, gb, wb, rb, ob, K, N, eps, s)));
      } else {
        TFD_CMAX_SWITCH(K, (launch_gemv<kC, 2, kPlain, kStore>(xb, gb, wb, rb, ob, K, N, eps, s)));
      }
      break;
    case TFD_EPI_RESID:
      if (norm) {
        TFD_CMAX_SWITCH(K, (launch_gemv<kC, 2, kNorm, kResid>(xb, gb, wb, rb, ob, K, N, eps, s)));
      } else {
        TFD_CMAX_SWITCH(K, (launch_gemv<kC, 2, kPlain, kResid>(xb, gb, wb, rb, ob, K, N, eps, s)));
      }
      break;
    case TFD_EPI_SWIGLU:
      if (norm) {
        TFD_CMAX_SWITCH(K, (launch_gemv<kC, 4, kNorm, kSwiglu>(xb, gb, wb, rb, ob, K, N, eps, s)));
      } else {
        TFD_CMAX_SWITCH(K, (launch_gemv<kC, 4, kPlain, kSwiglu>(xb, gb, wb, rb, ob, K, N, eps, s)));
      }
      break;
    default:
      return fail(kBadArg, "gemv: epilogue %d", epilogue);
  }
  return launched("gemv");
}

int tfd_lm_head_argmax_bf16(const void* x, const void* gamma, const void* w, float* logits,
                            float* block_val, int32_t* block_idx, int K, int V, int nblocks,
                            float eps, void* stream) {
  if (!x || !gamma || !w || !logits || !block_val || !block_idx)
    return fail(kBadArg, "lm_head: null pointer");
  if (K <= 0 || K % 8 || V <= 0 || nblocks <= 0)
    return fail(kBadShape, "lm_head: K=%d, V=%d, nblocks=%d", K, V, nblocks);
  auto s = (hipStream_t)stream;
  TFD_CMAX_SWITCH(K, hipLaunchKernelGGL((k_lm_head_argmax<kC, 4>), dim3(nblocks), dim3(kBlock), 0,
                                        s, (const bf16*)x, (const bf16*)gamma, (const bf16*)w,
                                        logits, block_val, block_idx, K, V, eps));
  return launched("lm_head");
}

int tfd_argmax_finalize(const float* block_val, const int32_t* block_idx, int nblocks,
                        const int32_t* inp, const int32_t* prompt_len, int64_t* ids,
                        int32_t* pos, int32_t* sam, int nsteps, const void* table, void* hid,
                        int hidden, int vocab, int32_t* err, void* stream) {
  if (!block_val || !block_idx || !inp || !prompt_len || !ids || !pos || !sam || !table || !hid)
    return fail(kBadArg, "argmax_finalize: null pointer");
  if (nblocks <= 0 || nsteps <= 0 || hidden <= 0 || hidden % 8 || vocab <= 0)
    return fail(kBadShape, "argmax_finalize: nblocks=%d nsteps=%d hidden=%d vocab=%d", nblocks,
                nsteps, hidden, vocab);
  hipLaunchKernelGGL(k_argmax_finalize, dim3(1), dim3(1024), 0, (hipStream_t)stream, block_val,
                     block_idx, nblocks, inp, prompt_len, ids, pos, sam, nsteps,
                     (const bf16*)table, (bf16*)hid, hidden, vocab, err);
  return launched("argmax_finalize");
}

#define TFD_ATTN_SWITCH(D, G, CALL)                                        \
  if (D == 128 && G == 2) { constexpr int kD = 128, kG = 2; CALL; }        \
  else if (D == 64 && G == 2) { constexpr int kD = 64, kG = 2; CALL; }     \
  else if (D == 128 && G == 1) { constexpr int kD = 128, kG = 1; CALL; }   \
  else return fail(kUnsupported, "attention: head_dim=%d group=%d not built", D, G);

int tfd_attn_rope_scores_paged(const void* qkv, const void* gamma_q, const void* gamma_k,
                               const void* cos_table, const void* sin_table, int rope_rows,
                               const int32_t* rope_pos, const int32_t* cache_len,
                               const int32_t* page_table, int max_pages, void* k_pool,
                               void* v_pool, int num_pages, int heads, int kv_heads,
                               int head_dim, float scale, float eps, float* scores,
                               int score_stride, float* split_max, float* score_new, int nsplit,
                               int32_t* err, void* stream) {
  if (!qkv || !gamma_q || !gamma_k || !cos_table || !sin_table || !rope_pos || !cache_len ||
      !page_table || !k_pool || !v_pool || !scores || !split_max || !score_new)
    return fail(kBadArg, "attn_rope_scores: null pointer");
  if (kv_heads <= 0 || heads % kv_heads || nsplit <= 0 || max_pages <= 0 || num_pages <= 0)
    return fail(kBadShape, "attn_rope_scores: heads=%d kv_heads=%d nsplit=%d pages=%d/%d", heads,
                kv_heads, nsplit, max_pages, num_pages);
  if ((int64_t)nsplit * kSplit < (int64_t)max_pages * kPage || score_stride < nsplit * kSplit)
    return fail(kBadShape,
                "attn_rope_scores: nsplit=%d x %d must cover max_pages=%d x %d and score_stride=%d",
                nsplit, kSplit, max_pages, kPage, score_stride);
  const int G = heads / kv_heads;
  auto s = (hipStream_t)stream;
  TFD_ATTN_SWITCH(head_dim, G,
                  hipLaunchKernelGGL((k_attn_rope_scores<kD, kG>), dim3(nsplit, kv_heads),
                                     dim3(kBlock), 0, s, (const bf16*)qkv, (const bf16*)gamma_q,
                                     (const bf16*)gamma_k, (const bf16*)cos_table,
                                     (const bf16*)sin_table, rope_rows, rope_pos, cache_len,
                                     page_table, max_pages, (bf16*)k_pool, (bf16*)v_pool,
                                     num_pages, kv_heads, scale, eps, scores, score_stride,
                                     split_max, score_new, err));
  return launched("attn_rope_scores");
}

int tfd_attn_pv_combine_paged(const void* qkv, const int32_t* cache_len,
                              const int32_t* page_table, int max_pages, const void* v_pool,
                              int num_pages, int heads, int kv_heads, int head_dim,
                              const float* scores, int score_stride, const float* split_max,
                              const float* score_new, float* part_sum, float* part_out,
                              int nsplit, int32_t* counters, void* attn_out, int32_t* err,
                              void* stream) {
  if (!qkv || !cache_len || !page_table || !v_pool || !scores || !split_max || !score_new ||
      !part_sum || !part_out || !counters || !attn_out)
    return fail(kBadArg, "attn_pv_combine: null pointer");
  if (kv_heads <= 0 || heads % kv_heads || nsplit <= 0 || max_pages <= 0 || num_pages <= 0)
    return fail(kBadShape, "attn_pv_combine: heads=%d kv_heads=%d nsplit=%d", heads, kv_heads,
                nsplit);
  if ((int64_t)nsplit * kSplit < (int64_t)max_pages * kPage || score_stride < nsplit * kSplit)
    return fail(kBadShape, "attn_pv_combine: nsplit=%d does not cover max_pages=%d", nsplit,
                max_pages);
  const int G = heads / kv_heads;
  auto s = (hipStream_t)stream;
  TFD_ATTN_SWITCH(head_dim, G,
                  hipLaunchKernelGGL((k_attn_pv_combine<kD, kG>), dim3(nsplit, kv_heads),
                                     dim3(kBlock), 0, s, (const bf16*)qkv, cache_len, page_table,
                                     max_pages, (const bf16*)v_pool, num_pages, kv_heads, scores,
                                     score_stride, split_max, score_new, part_sum, part_out,
                                     counters, (bf16*)attn_out, err));
  return launched("attn_pv_combine");
}

int tfd_decode_persistent_grid(void) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  return cus;
}

int tfd_decode_persistent(const TfdDecodeArgs* args, int steps, int nblocks, void* stream) {
  if (!args) return fail(kBadArg, "decode_persistent: null args");
  const TfdDecodeArgs& a = *args;
  if (!a.layers || !a.w_embed || !a.w_head || !a.gamma_final || !a.cos_table || !a.sin_table ||
      !a.page_table || !a.x_hid || !a.x_h1 || !a.x_qkv || !a.x_attn || !a.x_mid || !a.x_smax ||
      !a.x_psum || !a.x_pout || !a.x_best || !a.scores || !a.score_new || !a.logits || !a.ids ||
      !a.pos || !a.inp || !a.prompt_len || !a.sam || !a.err)
    return fail(kBadArg, "decode_persistent: null pointer in args");
  if (steps < 0) return fail(kBadArg, "decode_persistent: steps=%d", steps);
  if (steps == 0) return 0;
  if (a.n_layers <= 0 || a.kv_heads <= 0 || a.heads % a.kv_heads || a.hidden % 8 ||
      a.intermediate % 8 || a.vocab <= 0 || a.nsteps <= 0)
    return fail(kBadShape, "decode_persistent: bad model shape");
  if ((uint64_t)a.epoch + (uint64_t)steps * (uint64_t)(a.n_layers + 1) >= 0xffffffffull)
    return fail(kBadArg, "decode_persistent: epoch %u + %d steps passes 2^32: zero the exchange "
                "buffers and restart the epoch at 0", a.epoch, steps);
  if (a.heads * a.head_dim != a.hidden)
    return fail(kUnsupported, "decode_persistent: needs hidden == heads * head_dim (%d vs %d)",
                a.hidden, a.heads * a.head_dim);
  if ((int64_t)a.nsplit * kSplit < (int64_t)a.max_pages * kPage ||
      a.score_stride < a.nsplit * kSplit || a.num_pages <= 0)
    return fail(kBadShape, "decode_persistent: nsplit=%d does not cover max_pages=%d", a.nsplit,
                a.max_pages);
  const int grid = nblocks > 0 ? nblocks : tfd_decode_persistent_grid();
  if (grid <= 0) return fail(kUnsupported, "decode_persistent: no device");
  if ((int64_t)a.nsplit * a.kv_heads > 4LL * grid)
    return fail(kUnsupported, "decode_persistent: %d attention items exceed 4 per block of %d",
                a.nsplit * a.kv_heads, grid);
  const int G = a.heads / a.kv_heads;
  const int ch = cmax_for(a.hidden), ci = cmax_for(a.intermediate);
  const void* fn = nullptr;
  if (ch == 4 && ci == 12 && a.head_dim == 128 && G == 2)
    fn = reinterpret_cast<const void*>(&k_decode_persistent<4, 12, 128, 2>);
  else if (ch == 1 && ci == 2 && a.head_dim == 64 && G == 2)
    fn = reinterpret_cast<const void*>(&k_decode_persistent<1, 2, 64, 2>);
  else
    return fail(kUnsupported, "decode_persistent: no instance for hidden=%d inter=%d D=%d G=%d",
                a.hidden, a.intermediate, a.head_dim, G);
  int per_cu = 0, cus = tfd_decode_persistent_grid();
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kBlock, 0);
  if (e != hipSuccess) return fail((int)e, "decode_persistent: occupancy query failed");
  if (grid > per_cu * cus)
    return fail(kUnsupported, "decode_persistent: %d blocks cannot be co-resident (%d x %d)",
                grid, per_cu, cus);
  TfdDecodeArgs karg = a;
  int ksteps = steps;
  void* kargs[] = {&karg, &ksteps};
  // The grid fits the device at once (checked above), which is all the kernel
  // needs; the cooperative launch makes the runtime guarantee it.
  // TFD_PLAIN_LAUNCH=1 uses an ordinary launch instead, for profilers that do
  // not handle cooperative launches.
  static const bool plain = [] {
    const char* v = getenv("TFD_PLAIN_LAUNCH");
    return v && v[0] == '1';
  }();
  if (plain)
    e = hipLaunchKernel(fn, dim3(grid), dim3(kBlock), kargs, 0, (hipStream_t)stream);
  else
    e = hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kBlock), kargs, 0, (hipStream_t)stream);
  if (e != hipSuccess) return fail((int)e, "decode_persistent: launch failed: %s",
                                   hipGetErrorString(e));
  return launched("decode_persistent");
}

}  // extern "C"
