// Phase bodies of the decode step, shared by the per-kernel entries and the
// persistent decode kernel.  Each takes the index of the "virtual block" it
// plays (what blockIdx would be in a one-kernel-per-phase launch) so the two
// launch styles run the same code on the same data partition and produce the
// same bits.  All phases use 256-thread blocks.
//
// Every value a phase reads that another block of the same launch may have
// written -- activations, scores, partials, the KV cache, the position -- is
// read with device-coherent loads, and every such value is written with
// device-coherent stores (decode_common.h), so the persistent kernel's grid
// barriers need no cache writeback or invalidation.  Weights, norm scales, rope
// tables and the page table are read-only for a launch and use plain loads.
#pragma once

#include "decode_common.h"

namespace tfd {

constexpr float kNegInf = -__builtin_huge_valf();

enum Prologue { kPlain = 0, kNorm = 1 };
enum Epilogue { kStore = 0, kResid = 1, kSwiglu = 2 };

// ---------------------------------------------------------------------------
// Row-dot GEMV with fused prologue / epilogue.  One wave owns kR consecutive
// output rows; a block is 4 waves.  Every wave normalises x itself (a few KB)
// so no block waits on another.  Split into issue (the weight loads, which
// depend on nothing) and finish (x, norm, dot, epilogue) so a caller can put
// the weight loads in flight before it waits for x to exist.
// ---------------------------------------------------------------------------
template <int kCmax, int kR>
__device__ __forceinline__ void gemv_issue(int vb, const bf16* __restrict__ W, int K, int N,
                                           u32x4 (&w)[kR][kCmax]) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row0 = ((int64_t)vb * kWavesPerBlock + wave) * kR;
  if (row0 >= N) {
    // always define the tile: an undefined tile would be merged with the
    // previous one and kept live across the caller's loop
#pragma unroll
    for (int r = 0; r < kR; ++r)
#pragma unroll
      for (int i = 0; i < kCmax; ++i) w[r][i] = u32x4{0u, 0u, 0u, 0u};
    return;
  }
  const int nvalid = (int)((N - row0) < kR ? (N - row0) : kR);
  load_rows<kCmax, kR>(W, K, K / 8, row0, nvalid, lane, w);
}

template <int kCmax, int kR, int kPro, int kEpi>
__device__ __forceinline__ void gemv_finish(int vb, const bf16* __restrict__ x,
                                            const bf16* __restrict__ gamma,
                                            const bf16* __restrict__ resid,
                                            bf16* __restrict__ out, int K, int N, float eps,
                                            const u32x4 (&xin)[kCmax], const u32x4 (&gr)[kCmax],
                                            const u32x4 (&w)[kR][kCmax]) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row0 = ((int64_t)vb * kWavesPerBlock + wave) * kR;
  if (row0 >= N) return;
  const int nvalid = (int)((N - row0) < kR ? (N - row0) : kR);
  u32x4 xr[kCmax];
#pragma unroll
  for (int i = 0; i < kCmax; ++i) xr[i] = xin[i];
  if (kPro == kNorm) rms_norm_apply<kCmax>(xr, gr, K, eps);
  float acc[kR];
  dot_loaded<kCmax, kR>(w, xr, acc);

  if (kEpi == kSwiglu) {
    // rows come as (gate_n, up_n) pairs: mlp(), model.py:230-233
#pragma unroll
    for (int p = 0; p < kR / 2; ++p) {
      if (lane == p && 2 * p + 1 < nvalid) {
        const float g = rbf(acc[2 * p]);
        const float u = rbf(acc[2 * p + 1]);
        const float a = rbf(silu_f(g));
        coh_st_bf16(out, (uint32_t)(row0 / 2 + p), f2bf(a * u));
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      if (lane == r && r < nvalid) {
        const float y = rbf(acc[r]);
        if (kEpi == kResid)
          coh_st_bf16(out, (uint32_t)(row0 + r),
                      f2bf(bf2f(coh_ld_bf16(resid, (uint32_t)(row0 + r))) + y));
        else
          coh_st_bf16(out, (uint32_t)(row0 + r), f2bf(y));
      }
    }
  }
}

// x (and gamma) for a finish: issued before the weights when both are loaded
// in one go, because memory counters retire in order.  x is read through the
// caches: every wave of the grid reads it, and a device-scope read would send
// them all to the few memory channels holding it.  The caller guarantees that
// no cache holds a stale copy (a fresh address per layer, and the persistent
// kernel invalidates L2 at every step boundary).
template <int kCmax, int kPro>
__device__ __forceinline__ void gemv_load_x(const bf16* __restrict__ x,
                                            const bf16* __restrict__ gamma, int K,
                                            u32x4 (&xr)[kCmax], u32x4 (&gr)[kCmax]) {
  const int lane = threadIdx.x & (kWave - 1);
  load_x<kCmax>(x, K / 8, lane, xr);
  if (kPro == kNorm) load_x<kCmax>(gamma, K / 8, lane, gr);
}

template <int kCmax, int kR, int kPro, int kEpi>
__device__ __forceinline__ void gemv_phase(int vb, const bf16* __restrict__ x,
                                           const bf16* __restrict__ gamma,
                                           const bf16* __restrict__ W,
                                           const bf16* __restrict__ resid,
                                           bf16* __restrict__ out, int K, int N, float eps) {
  const int wave = threadIdx.x / kWave;
  if (((int64_t)vb * kWavesPerBlock + wave) * kR >= N) return;
  u32x4 xr[kCmax], gr[kCmax];
  gemv_load_x<kCmax, kPro>(x, gamma, K, xr, gr);
  u32x4 w[kR][kCmax];
  gemv_issue<kCmax, kR>(vb, W, K, N, w);
  gemv_finish<kCmax, kR, kPro, kEpi>(vb, x, gamma, resid, out, K, N, eps, xr, gr, w);
}

// ---------------------------------------------------------------------------
// lm_head (model.py:300-305) with the final norm folded in and a per-block
// greedy pick: logits are rounded to bf16 (the HIR declares them bf16) and the
// block keeps the largest, lowest index on ties (torch.argmax's rule,
// generation.py:24-26).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

template <int kCmax, int kR>
__device__ __forceinline__ void lm_head_phase(int vb, int nvb, const bf16* __restrict__ x,
                                              const bf16* __restrict__ gamma,
                                              const bf16* __restrict__ W,
                                              float* __restrict__ logits, float* __restrict__ bv,
                                              int* __restrict__ bi, int K, int V, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nch = K / 8;
  u32x4 xr[kCmax];
  rms_norm_x<kCmax>(x, gamma, K, eps, lane, xr);
  float best = kNegInf;
  int besti = 0x7fffffff;
  const int64_t stride = (int64_t)nvb * kWavesPerBlock * kR;
  for (int64_t row0 = ((int64_t)vb * kWavesPerBlock + wave) * kR; row0 < V; row0 += stride) {
    const int nvalid = (int)((V - row0) < kR ? (V - row0) : kR);
    float acc[kR];
    dot_rows<kCmax, kR>(W, K, nch, row0, nvalid, xr, lane, acc);
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
  // every lane of a wave holds the same (best, besti); reduce across waves
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
    coh_stf(&bv[vb], b);
    coh_sti(&bi[vb], i);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// The step's last node (fast/kernels.py:591-637 does the same job): global
// argmax over the block picks, record it at Sam[pos], feed the next prompt token
// while the prompt lasts and the pick after, advance pos, and stage the next
// token's embedding row as the next step's hidden state.  One block.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void finalize_phase(const float* __restrict__ bv,
                                               const int* __restrict__ bi, int nb,
                                               const int* __restrict__ inp,
                                               const int* __restrict__ plen,
                                               int64_t* __restrict__ ids, int* __restrict__ pos,
                                               int* __restrict__ sam, int nsteps,
                                               const bf16* __restrict__ table,
                                               bf16* __restrict__ hid, int hidden, int vocab,
                                               int* err) {
  const int tid = threadIdx.x;
  float b = kNegInf;
  int i = 0x7fffffff;
  for (int k = tid; k < nb; k += blockDim.x) {
    const float v = coh_ldf(&bv[k]);
    const int ix = coh_ldi(&bi[k]);
    if (better(v, ix, b, i)) {
      b = v;
      i = ix;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ob = __shfl_xor(b, m, kWave);
    const int oi = __shfl_xor(i, m, kWave);
    if (better(ob, oi, b, i)) {
      b = ob;
      i = oi;
    }
  }
  __shared__ float sv[16];
  __shared__ int si[16];
  __shared__ int next_s;
  const int lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  if (lane == 0) {
    sv[wave] = b;
    si[wave] = i;
  }
  __syncthreads();
  if (tid == 0) {
    float bb = sv[0];
    int ii = si[0];
    for (int w = 1; w < nw; ++w)
      if (better(sv[w], si[w], bb, ii)) {
        bb = sv[w];
        ii = si[w];
      }
    if (ii < 0 || ii >= vocab) ii = 0;  // all-NaN row: no pick exists
    const int p = coh_ldi(pos);
    int next = ii;
    if (p < 0 || p >= nsteps) {
      raise_error(err, kErrStepRange);
    } else {
      sam[p] = ii;
      if (p + 1 < plen[0] && p + 1 < nsteps) next = inp[p + 1];
    }
    if (next < 0 || next >= vocab) {
      raise_error(err, kErrTokenRange);
      next = 0;
    }
    coh_sti64(ids, next);
    coh_sti(pos, p + 1);
    next_s = next;
  }
  __syncthreads();
  const bf16* row = table + (int64_t)next_s * hidden;
  for (int c = tid; c < hidden / 8; c += blockDim.x)
    coh_st16(hid, (uint32_t)c * 16u, load16(row + (int64_t)c * 8));
}

// ---------------------------------------------------------------------------
// Attention over the paged cache, two phases per layer (model.py:172-212).
// Virtual block (split, kv head h) owns kSplit context positions of one kv head
// and its group of G query heads.  The K and V tiles a block reads depend only
// on the position and the page table, so they are issued separately (KTile /
// VTile) and a caller can put them in flight before it waits for the QKV
// projection.  Every load is unconditional from a clamped, in-bounds address and
// masked afterwards: a load under a divergent branch gets waited on inside it.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t page_row(int page, int j, int kv_heads, int h, int D) {
  return (((int64_t)page * kv_heads + h) * kPage + (j % kPage)) * D;
}

template <int D>
struct AttnShape {
  static constexpr int kLpp = D / 8;                        // lanes per position (16-byte chunks)
  static constexpr int kPpw = kWave / kLpp;                 // positions per wave, scores pass
  static constexpr int kKPasses = kSplit / (kWavesPerBlock * kPpw);
  static constexpr int kGroups = kBlock / kLpp;             // position groups, P.V pass
  static constexpr int kVPasses = kSplit / kGroups;
  static_assert(kKPasses * kWavesPerBlock * kPpw == kSplit, "split tiles the scores pass");
  static_assert(kVPasses * kGroups == kSplit, "split tiles the P.V pass");
};

template <int D>
struct KTile {
  int pg[AttnShape<D>::kKPasses];
  u32x4 t[AttnShape<D>::kKPasses];
};
template <int D>
struct VTile {
  int pg[AttnShape<D>::kVPasses];
  u32x4 t[AttnShape<D>::kVPasses];
};

// position a thread reads in pass p of each pass layout
template <int D>
__device__ __forceinline__ int k_pos(int j0, int p) {
  using A = AttnShape<D>;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  return j0 + p * kWavesPerBlock * A::kPpw + wave * A::kPpw + lane / A::kLpp;
}
template <int D>
__device__ __forceinline__ int v_pos(int j0, int p) {
  using A = AttnShape<D>;
  return j0 + (int)threadIdx.x / A::kLpp + p * A::kGroups;
}

// K rows of split `split` (positions j < P are the ones used).  A split that
// holds no prior position issues nothing.
template <int D>
__device__ __forceinline__ void k_tile_issue(int split, int h, int P, const int* page_table,
                                             int max_pages, const bf16* kpool, int num_pages,
                                             int kv_heads, KTile<D>& kt) {
  using A = AttnShape<D>;
  const int j0 = split * kSplit;
  const int ch = (threadIdx.x & (kWave - 1)) % A::kLpp;
#pragma unroll
  for (int p = 0; p < A::kKPasses; ++p) {
    kt.pg[p] = -1;
    kt.t[p] = u32x4{0u, 0u, 0u, 0u};
  }
  if (j0 >= P) return;
#pragma unroll
  for (int p = 0; p < A::kKPasses; ++p) {
    const int j = k_pos<D>(j0, p);
    kt.pg[p] = page_table[j / kPage < max_pages ? j / kPage : max_pages - 1];
  }
#pragma unroll
  for (int p = 0; p < A::kKPasses; ++p) {
    const int j = k_pos<D>(j0, p);
    const bool bad = kt.pg[p] < 0 || kt.pg[p] >= num_pages;
    kt.t[p] = coh_ld16(kpool, (uint32_t)(page_row(bad ? 0 : kt.pg[p], j, kv_heads, h, D) +
                                         ch * 8) * 2u);
  }
}

template <int D>
__device__ __forceinline__ void v_tile_issue(int split, int h, int P, const int* page_table,
                                             int max_pages, const bf16* vpool, int num_pages,
                                             int kv_heads, VTile<D>& vt) {
  using A = AttnShape<D>;
  const int j0 = split * kSplit;
  const int ch = (int)threadIdx.x % A::kLpp;
#pragma unroll
  for (int p = 0; p < A::kVPasses; ++p) {
    vt.pg[p] = -1;
    vt.t[p] = u32x4{0u, 0u, 0u, 0u};
  }
  if (j0 >= P) return;
#pragma unroll
  for (int p = 0; p < A::kVPasses; ++p) {
    const int j = v_pos<D>(j0, p);
    vt.pg[p] = page_table[j / kPage < max_pages ? j / kPage : max_pages - 1];
  }
#pragma unroll
  for (int p = 0; p < A::kVPasses; ++p) {
    const int j = v_pos<D>(j0, p);
    const bool bad = vt.pg[p] < 0 || vt.pg[p] >= num_pages;
    vt.t[p] = coh_ld16(vpool, (uint32_t)(page_row(bad ? 0 : vt.pg[p], j, kv_heads, h, D) +
                                         ch * 8) * 2u);
  }
}

// ---------------------------------------------------------------------------
// Part 1 (model.py:172-198).  Each block rebuilds its kv head's group of query
// vectors and the new key from the bf16 QKV projection: per-head RMS, RoPE at
// rp, q_s = bf16(q_rope * scale).  Split 0 writes this token's key and value
// into the paged cache at position P and scores the new key; every block scores
// its own positions of the prior context,
//   s_j = bf16( sum_d bf16(q_s[d] * K[j][d]) ),
// and records the split's max per query head.
// ---------------------------------------------------------------------------
template <int D, int G>
__device__ __forceinline__ void attn_scores_phase(
    int split, int h, const bf16* __restrict__ qkv, const bf16* __restrict__ gq,
    const bf16* __restrict__ gk, const bf16* __restrict__ cos_t, const bf16* __restrict__ sin_t,
    int rope_rows, int rp, int P, const int* __restrict__ page_table, int max_pages,
    bf16* __restrict__ kpool, bf16* __restrict__ vpool, int num_pages, int kv_heads, float scale,
    float eps, float* __restrict__ S, int s_stride, float* __restrict__ smax,
    float* __restrict__ snew, const KTile<D>& kt, int* err) {
  using A = AttnShape<D>;
  constexpr int kHalf = D / 2;
  constexpr int kLpp = A::kLpp;
  static_assert(kHalf <= kWave, "one wave holds a head as (d, d + D/2) lane pairs");
  static_assert(G + 1 <= kWavesPerBlock, "one wave per vector");
  const int heads = kv_heads * G;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int j0 = split * kSplit;
  const int ch = lane % kLpp;

  if (split != 0 && j0 >= P) {
    if (tid < G) coh_stf(&smax[split * heads + h * G + tid], kNegInf);
    return;
  }
  if (P < 0 || P >= max_pages * kPage || rp < 0 || rp >= rope_rows) {
    if (tid == 0) raise_error(err, kErrPosRange);
    if (tid < G) {
      coh_stf(&smax[split * heads + h * G + tid], kNegInf);
      if (split == 0) coh_stf(&snew[h * G + tid], 0.f);
    }
    return;
  }
  // ---- this head's QKV slice, gammas and rope rows (one round trip)
  const int v = wave;                     // vector this wave normalises (G queries + 1 key)
  const bool has_vec = v < G + 1;
  const bool isq = v < G;
  const bool act = has_vec && lane < kHalf;
  const int li = lane < kHalf ? lane : 0;
  const uint32_t src = isq ? (uint32_t)((h * G + (isq ? v : 0)) * D) : (uint32_t)(heads * D + h * D);
  const bf16* gam = isq ? gq : gk;
  const bf16 rx0 = qkv[src + li], rx1 = qkv[src + li + kHalf];
  const bf16 rg0 = gam[li], rg1 = gam[li + kHalf];
  const bf16 rc0 = cos_t[(int64_t)rp * D + li], rs0 = sin_t[(int64_t)rp * D + li];
  const bf16 rc1 = cos_t[(int64_t)rp * D + li + kHalf], rs1 = sin_t[(int64_t)rp * D + li + kHalf];
  const int page_new = page_table[P / kPage];
  const int jend = (j0 + kSplit < P) ? j0 + kSplit : P;
  const float x0 = act ? bf2f(rx0) : 0.f, x1 = act ? bf2f(rx1) : 0.f;
  const float g0 = bf2f(rg0), g1 = bf2f(rg1);
  const float c0 = bf2f(rc0), s0 = bf2f(rs0), c1 = bf2f(rc1), s1 = bf2f(rs1);

  __shared__ float qs[G][D];
  __shared__ float kn[D];
  __shared__ float wmax[kWavesPerBlock][G];

  // ---- q group and the new key: RMS over D, bf16, * gamma, RoPE, (q) * scale
  if (has_vec) {
    float ss = x0 * x0;
    ss += x1 * x1;
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
    if (act) {
      const float n0 = rbf(rbf(x0 * r) * g0);
      const float n1 = rbf(rbf(x1 * r) * g1);
      // rope.py:154-162: x*cos + rotate_half(x)*sin, rotate_half = (-x2, x1)
      const float o0 = rbf(n0 * c0 + (-n1) * s0);
      const float o1 = rbf(n1 * c1 + n0 * s1);
      if (isq) {
        qs[v][lane] = rbf(o0 * scale);
        qs[v][lane + kHalf] = rbf(o1 * scale);
      } else {
        kn[lane] = o0;
        kn[lane + kHalf] = o1;
      }
    }
  }
  __syncthreads();

  if (split == 0) {
    // this token's entry goes to the cache at P (fast/kernels.py:385-409)
    if (page_new < 0 || page_new >= num_pages) {
      if (tid == 0) raise_error(err, kErrPageRange);
    } else {
      const int64_t off = page_row(page_new, P, kv_heads, h, D);
      const uint32_t vsrc = (uint32_t)(heads * D + kv_heads * D + h * D);
      for (int d = tid; d < D; d += kBlock) {
        coh_st_bf16(kpool, (uint32_t)(off + d), f2bf(kn[d]));
        coh_st_bf16(vpool, (uint32_t)(off + d), qkv[vsrc + d]);
      }
    }
    // score of the new key (score_new, model.py:198)
    if (wave < G) {
      float a = 0.f;
      if (lane < kHalf) {
        a = rbf(qs[wave][lane] * kn[lane]);
        a += rbf(qs[wave][lane + kHalf] * kn[lane + kHalf]);
      }
      a = wave_sum(a);
      if (lane == 0) coh_stf(&snew[h * G + wave], rbf(a));
    }
  }

  // ---- scores over this split of the prior context
  float qv[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[g][e] = qs[g][ch * 8 + e];
  float mymax[G];
#pragma unroll
  for (int g = 0; g < G; ++g) mymax[g] = kNegInf;
  bool page_ok = true;
#pragma unroll
  for (int p = 0; p < A::kKPasses; ++p) {
    const int j = k_pos<D>(j0, p);
    const bool bad = kt.pg[p] < 0 || kt.pg[p] >= num_pages;
    if (j < jend && bad) page_ok = false;
    const bool valid = j < jend && !bad;
    const uint32_t kw[4] = {kt.t[p].x, kt.t[p].y, kt.t[p].z, kt.t[p].w};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a += rbf(qv[g][2 * e] * bf_lo(kw[e]));
        a += rbf(qv[g][2 * e + 1] * bf_hi(kw[e]));
      }
      a = group_sum<kLpp>(a);
      const float sc = rbf(a);
      if (valid) {
        if (ch == 0) coh_stf(&S[(int64_t)(h * G + g) * s_stride + j], sc);
        mymax[g] = fmaxf(mymax[g], sc);
      }
    }
  }
  if (!page_ok) raise_error(err, kErrPageRange);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = wave_max(mymax[g]);
    if (lane == 0) wmax[wave][g] = m;
  }
  __syncthreads();
  if (tid < G) {
    float m = wmax[0][tid];
    for (int w = 1; w < kWavesPerBlock; ++w) m = fmaxf(m, wmax[w][tid]);
    coh_stf(&smax[split * heads + h * G + tid], m);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Part 2 (model.py:200-212).  With the joint peak M = max(split maxima, score_new):
//   p_j = bf16(exp(bf16(s_j - M)))
//   per split: sum_j p_j and sum_j bf16(p_j * V[j][d]) in f32
// The last block of a kv head to finish merges every split, in split order:
//   total    = bf16(bf16(sum p) + p_new)
//   weighted = bf16(bf16(sum pV) + bf16(p_new * v_new))
//   attn     = bf16(weighted / total)
// "Last" is decided by a per-head counter; partials are written and read
// device-coherently, and each wave waits for its own stores before the block
// counts itself in, so the merging block sees every split.  The merging block
// stages the partials through LDS with coalesced 16-byte loads.
// ---------------------------------------------------------------------------
template <int D, int G>
__device__ __forceinline__ void attn_pv_phase(
    int split, int h, int nsplit, const bf16* __restrict__ qkv, int P,
    const int* __restrict__ page_table, int max_pages, const bf16* __restrict__ vpool,
    int num_pages, int kv_heads, const float* __restrict__ S, int s_stride,
    const float* __restrict__ smax, const float* __restrict__ snew, float* part_sum,
    float* part_out, int* counters, bf16* __restrict__ attn_out, const VTile<D>& vt, int* err) {
  using A = AttnShape<D>;
  constexpr int kLpp = A::kLpp;
  constexpr int kGroups = A::kGroups;
  constexpr int kOut = G * D;                         // outputs of the head group
  static_assert(kSplit == kWave, "one wave sums one head's split of p");
  static_assert(G <= kWavesPerBlock, "one wave per query head of the group");
  static_assert(kOut % 4 == 0 && kOut <= kBlock, "one thread per output");
  const int heads = kv_heads * G;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int ch = tid % kLpp, jo = tid / kLpp;
  const int j0 = split * kSplit;
  (void)max_pages;
  (void)page_table;
  (void)vpool;

  if (P < 0 || P >= max_pages * kPage) P = 0;  // part 1 already raised the flag
  const int nact = (P + kSplit - 1) / kSplit;
  const int participants = nact > 0 ? nact : 1;
  if (split >= participants) return;
  const int jend = (j0 + kSplit < P) ? j0 + kSplit : P;

  // ---- this split's scores, every split's max, the new-key scores
  const int wg = wave < G ? wave : 0;
  const float sn = coh_ldf(&snew[h * G + wg]);
  const float sj_raw = coh_ldf(&S[(int64_t)(h * G + wg) * s_stride + j0 + lane]);
  float mx = kNegInf;
  for (int s0 = 0; s0 < nact; s0 += kWave) {
    const int s = s0 + lane;
    const float m = coh_ldf(&smax[(s < nsplit ? s : nsplit - 1) * heads + h * G + wg]);
    if (s < nact) mx = fmaxf(mx, m);
  }
  const float sj = (j0 + lane < jend) ? sj_raw : kNegInf;

  __shared__ float M[G];
  __shared__ float p[G][kSplit];
  __shared__ float red[kGroups][kOut];
  __shared__ float psums[kGroups][G];
  __shared__ int is_last;

  if (wave < G) {
    const float m = fmaxf(wave_max(mx), sn);
    if (lane == 0) M[wave] = m;
    const float pj = (j0 + lane < jend) ? rbf(expf(rbf(sj - m))) : 0.f;
    p[wave][lane] = pj;
    const float s = wave_sum(pj);
    if (lane == 0) coh_stf(&part_sum[split * heads + h * G + wave], s);
  }
  __syncthreads();
  {
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    bool page_ok = true;
#pragma unroll
    for (int q = 0; q < A::kVPasses; ++q) {
      const int jj = jo + q * kGroups;
      const bool bad = vt.pg[q] < 0 || vt.pg[q] >= num_pages;
      if (j0 + jj < jend && bad) page_ok = false;
      const u32x4 t = (j0 + jj < jend && !bad) ? vt.t[q] : u32x4{0u, 0u, 0u, 0u};
      const uint32_t vw[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pj = p[g][jj];          // 0 past the end: adds exact zeros
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[g][2 * e] += rbf(pj * bf_lo(vw[e]));
          acc[g][2 * e + 1] += rbf(pj * bf_hi(vw[e]));
        }
      }
    }
    if (!page_ok) raise_error(err, kErrPageRange);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[jo][g * D + ch * 8 + e] = acc[g][e];
  }
  __syncthreads();
  for (int o = tid; o < kOut; o += kBlock) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < kGroups; ++q) s += red[q][o];
    coh_stf(&part_out[((int64_t)split * heads + h * G) * D + o], s);
  }
  // ---- the last block of this kv head merges the splits
  stores_done();
  __syncthreads();
  if (tid == 0) {
    const int ticket = atomicAdd(&counters[h], 1);
    is_last = (ticket == participants - 1);
  }
  __syncthreads();
  if (!is_last) return;
  // stage up to kGroups splits at a time: coalesced 16-byte device-coherent loads
  constexpr int kVecPerSplit = kOut / 4;
  constexpr int kIters = (kGroups * kVecPerSplit + kBlock - 1) / kBlock;
  float sv = 0.f, sp = 0.f;
  for (int c0 = 0; c0 < nact; c0 += kGroups) {
    const int nc = (nact - c0) < kGroups ? (nact - c0) : kGroups;
    u32x4 v[kIters];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int idx = tid + it * kBlock;
      const int s = idx / kVecPerSplit < nc ? idx / kVecPerSplit : nc - 1;
      const int q4 = idx % kVecPerSplit;
      v[it] = coh_ld16(part_out,
                       (uint32_t)((((int64_t)(c0 + s) * heads + h * G) * D + q4 * 4) * 4));
    }
    float ps = 0.f;
    if (tid < nc * G) ps = coh_ldf(&part_sum[(c0 + tid / G) * heads + h * G + tid % G]);
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int idx = tid + it * kBlock;
      if (idx / kVecPerSplit < nc) {
        float* dst = &red[idx / kVecPerSplit][(idx % kVecPerSplit) * 4];
        dst[0] = __uint_as_float(v[it].x);
        dst[1] = __uint_as_float(v[it].y);
        dst[2] = __uint_as_float(v[it].z);
        dst[3] = __uint_as_float(v[it].w);
      }
    }
    if (tid < nc * G) psums[tid / G][tid % G] = ps;
    __syncthreads();
    if (tid < kOut) {
      for (int s = 0; s < nc; ++s) {
        sv += red[s][tid];
        sp += psums[s][tid / D];
      }
    }
    __syncthreads();
  }
  if (tid < kOut) {
    const int g = tid / D, d = tid % D;
    const uint32_t vnew = (uint32_t)(heads * D + kv_heads * D + h * D);
    const float pn = rbf(expf(rbf(coh_ldf(&snew[h * G + g]) - M[g])));
    const float total = rbf(rbf(sp) + pn);
    const float weighted = rbf(rbf(sv) + rbf(pn * bf2f(qkv[vnew + d])));
    coh_st_bf16(attn_out, (uint32_t)((h * G + g) * D + d), f2bf(weighted / total));
  }
  if (tid == 0) atomicExch(&counters[h], 0);
  __syncthreads();
}

}  // namespace tfd
