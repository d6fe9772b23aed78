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

#include "decode_common.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

using namespace tfd;

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

enum Prologue { kPlain = 0, kNorm = 1 };
enum Epilogue { kStore = 0, kResid = 1, kSwiglu = 2 };

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
// Row-dot GEMV with fused prologue / epilogue.  One wave owns kR consecutive
// output rows; a block is 4 waves.  Every wave normalises x itself (a few KB
// from L2) so no block waits on another.
// ---------------------------------------------------------------------------
template <int kCmax, int kR, int kPro, int kEpi>
__global__ __launch_bounds__(kBlock) void k_gemv(const bf16* __restrict__ x,
                                                 const bf16* __restrict__ gamma,
                                                 const bf16* __restrict__ W,
                                                 const bf16* __restrict__ resid,
                                                 bf16* __restrict__ out, int K, int N, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * kR;
  if (row0 >= N) return;
  const int nch = K / 8;
  u32x4 xr[kCmax];
  if (kPro == kNorm)
    rms_norm_x<kCmax>(x, gamma, K, eps, lane, xr);
  else
    load_x<kCmax>(x, nch, lane, xr);
  const int nvalid = (int)((N - row0) < kR ? (N - row0) : kR);
  float acc[kR];
  dot_rows<kCmax, kR>(W, K, nch, row0, nvalid, xr, lane, acc);

  if (kEpi == kSwiglu) {
    // rows come as (gate_n, up_n) pairs: mlp(), model.py:230-233
#pragma unroll
    for (int p = 0; p < kR / 2; ++p) {
      if (lane == p && 2 * p + 1 < nvalid) {
        const float g = rbf(acc[2 * p]);
        const float u = rbf(acc[2 * p + 1]);
        const float a = rbf(silu_f(g));
        out[row0 / 2 + p] = f2bf(a * u);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      if (lane == r && r < nvalid) {
        const float y = rbf(acc[r]);
        if (kEpi == kResid)
          out[row0 + r] = f2bf(bf2f(resid[row0 + r]) + y);
        else
          out[row0 + r] = f2bf(y);
      }
    }
  }
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
__global__ __launch_bounds__(kBlock) void k_lm_head_argmax(
    const bf16* __restrict__ x, const bf16* __restrict__ gamma, const bf16* __restrict__ W,
    float* __restrict__ logits, float* __restrict__ bv, int* __restrict__ bi, int K, int V,
    float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nch = K / 8;
  u32x4 xr[kCmax];
  rms_norm_x<kCmax>(x, gamma, K, eps, lane, xr);
  float best = kNegInf;
  int besti = 0x7fffffff;
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock * kR;
  for (int64_t row0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * kR; row0 < V;
       row0 += stride) {
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
    bv[blockIdx.x] = b;
    bi[blockIdx.x] = i;
  }
}

// ---------------------------------------------------------------------------
// The step's last node (fast/kernels.py:591-637 does the same job): global
// argmax over the block picks, record it at Sam[pos], feed the next prompt token
// while the prompt lasts and the pick after, advance pos, and stage the next
// token's embedding row as the next step's hidden state.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_argmax_finalize(
    const float* __restrict__ bv, const int* __restrict__ bi, int nb,
    const int* __restrict__ inp, const int* __restrict__ plen, int64_t* __restrict__ ids,
    int* __restrict__ pos, int* __restrict__ sam, int nsteps, const bf16* __restrict__ table,
    bf16* __restrict__ hid, int hidden, int vocab, int* err) {
  const int tid = threadIdx.x;
  float b = kNegInf;
  int i = 0x7fffffff;
  for (int k = tid; k < nb; k += blockDim.x)
    if (better(bv[k], bi[k], b, i)) {
      b = bv[k];
      i = bi[k];
    }
  // wave reduction of (value, index)
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
    const int p = pos[0];
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
    ids[0] = next;
    pos[0] = p + 1;
    next_s = next;
  }
  __syncthreads();
  const bf16* row = table + (int64_t)next_s * hidden;
  for (int c = tid; c < hidden / 8; c += blockDim.x)
    *reinterpret_cast<u32x4*>(hid + (int64_t)c * 8) = load16(row + (int64_t)c * 8);
}

// ---------------------------------------------------------------------------
// Attention, part 1 (self_attention, model.py:172-198).
// Grid (nsplit, kv_heads).  Each block rebuilds its kv head's group of query
// vectors and the new key from the bf16 QKV projection: per-head RMS, RoPE at
// rope_pos, q_s = bf16(q_rope * scale).  Split 0 writes this token's key and
// value into the paged cache at position cache_len and scores the new key;
// every block scores its own kSplit positions of the prior context:
//   s_j = bf16( sum_d bf16(q_s[d] * K[j][d]) )
// and records the split's max per query head.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t page_offset(const int* page_table, int j, int kv_heads,
                                               int h, int D, int num_pages, bool* ok) {
  const int page = page_table[j / kPage];
  if (page < 0 || page >= num_pages) {
    *ok = false;
    return 0;
  }
  return (((int64_t)page * kv_heads + h) * kPage + (j % kPage)) * D;
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
  constexpr int kHalf = D / 2;
  constexpr int kLpp = D / 8;             // lanes per position (one 16-byte chunk each)
  constexpr int kPpw = kWave / kLpp;      // positions per wave per pass
  static_assert(kHalf <= kWave, "one wave holds a head as (d, d + D/2) lane pairs");
  const int split = blockIdx.x, h = blockIdx.y;
  const int heads = kv_heads * G;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int P = cache_len[0];
  const int rp = rope_pos[0];
  const int j0 = split * kSplit;
  if (split != 0 && j0 >= P) {
    if (tid < G) smax[split * heads + h * G + tid] = kNegInf;
    return;
  }
  if (P < 0 || P >= max_pages * kPage || rp < 0 || rp >= rope_rows) {
    if (tid == 0) raise_error(err, kErrPosRange);
    if (tid < G) {
      smax[split * heads + h * G + tid] = kNegInf;
      if (split == 0) snew[h * G + tid] = 0.f;
    }
    return;
  }

  __shared__ float qs[G][D];
  __shared__ float kn[D];
  __shared__ float wmax[kWavesPerBlock][G];

  // ---- q group and the new key: RMS over D, bf16, * gamma, RoPE, (q) * scale
  for (int v = wave; v < G + 1; v += kWavesPerBlock) {
    const bool isq = v < G;
    const bf16* src = isq ? qkv + (int64_t)(h * G + v) * D : qkv + (int64_t)heads * D + h * D;
    const bf16* gam = isq ? gq : gk;
    const bool act = lane < kHalf;
    const float x0 = act ? bf2f(src[lane]) : 0.f;
    const float x1 = act ? bf2f(src[lane + kHalf]) : 0.f;
    float ss = x0 * x0;
    ss += x1 * x1;
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
    if (act) {
      const float n0 = rbf(rbf(x0 * r) * bf2f(gam[lane]));
      const float n1 = rbf(rbf(x1 * r) * bf2f(gam[lane + kHalf]));
      const float c0 = bf2f(cos_t[(int64_t)rp * D + lane]);
      const float s0 = bf2f(sin_t[(int64_t)rp * D + lane]);
      const float c1 = bf2f(cos_t[(int64_t)rp * D + lane + kHalf]);
      const float s1 = bf2f(sin_t[(int64_t)rp * D + lane + kHalf]);
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
    bool ok = true;
    const int64_t off = page_offset(page_table, P, kv_heads, h, D, num_pages, &ok);
    if (!ok) {
      if (tid == 0) raise_error(err, kErrPageRange);
    } else {
      const bf16* vsrc = qkv + (int64_t)heads * D + (int64_t)kv_heads * D + h * D;
      for (int d = tid; d < D; d += kBlock) {
        kpool[off + d] = f2bf(kn[d]);
        vpool[off + d] = vsrc[d];
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
      if (lane == 0) snew[h * G + wave] = rbf(a);
    }
  }

  // ---- scores over this split of the prior context
  const int jend = (j0 + kSplit < P) ? j0 + kSplit : P;
  const int sub = lane / kLpp, ch = lane % kLpp;
  float qv[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[g][e] = qs[g][ch * 8 + e];
  float mymax[G];
#pragma unroll
  for (int g = 0; g < G; ++g) mymax[g] = kNegInf;
  bool page_ok = true;
  for (int jb = j0 + wave * kPpw; jb < jend; jb += kWavesPerBlock * kPpw) {
    const int j = jb + sub;
    const bool valid = j < jend;
    u32x4 kv = u32x4{0u, 0u, 0u, 0u};
    if (valid) {
      bool ok = true;
      const int64_t off = page_offset(page_table, j, kv_heads, h, D, num_pages, &ok);
      if (ok)
        kv = load16(kpool + off + ch * 8);
      else
        page_ok = false;
    }
    const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
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
        if (ch == 0) S[(int64_t)(h * G + g) * s_stride + j] = sc;
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
    smax[split * heads + h * G + tid] = m;
  }
}

// ---------------------------------------------------------------------------
// Attention, part 2 (model.py:200-212).  Grid (nsplit, kv_heads).
// With the joint peak M = max(split maxima, score_new):
//   p_j = bf16(exp(bf16(s_j - M)))
//   per split: sum_j p_j and sum_j bf16(p_j * V[j][d]) in f32
// The last block of a kv head to finish merges every split (in split order):
//   total    = bf16(bf16(sum p) + p_new)
//   weighted = bf16(bf16(sum pV) + bf16(p_new * v_new))
//   attn     = bf16(weighted / total)
// ---------------------------------------------------------------------------
template <int D, int G>
__global__ __launch_bounds__(kBlock) void k_attn_pv_combine(
    const bf16* __restrict__ qkv, const int* __restrict__ cache_len,
    const int* __restrict__ page_table, int max_pages, const bf16* __restrict__ vpool,
    int num_pages, int kv_heads, const float* __restrict__ S, int s_stride,
    const float* __restrict__ smax, const float* __restrict__ snew, float* part_sum,
    float* part_out, int* counters, bf16* __restrict__ attn_out, int* err) {
  constexpr int kLpp = D / 8;
  constexpr int kGroups = kBlock / kLpp;   // position groups in the P.V pass
  static_assert(kSplit == kWave, "one wave sums one head's split of p");
  const int split = blockIdx.x, h = blockIdx.y;
  const int heads = kv_heads * G;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  int P = cache_len[0];
  if (P < 0 || P >= max_pages * kPage) P = 0;  // part 1 already raised the flag
  const int nact = (P + kSplit - 1) / kSplit;
  const int participants = nact > 0 ? nact : 1;
  if (split >= participants) return;

  __shared__ float M[G];
  __shared__ float p[G][kSplit];
  __shared__ float red[kGroups][G * D];
  __shared__ int is_last;

  if (tid < G) {
    float m = snew[h * G + tid];
    for (int s = 0; s < nact; ++s) m = fmaxf(m, smax[s * heads + h * G + tid]);
    M[tid] = m;
  }
  __syncthreads();
  const int j0 = split * kSplit;
  const int jend = (j0 + kSplit < P) ? j0 + kSplit : P;
  for (int idx = tid; idx < G * kSplit; idx += kBlock) {
    const int g = idx / kSplit, jj = idx % kSplit, j = j0 + jj;
    p[g][jj] = (j < jend) ? rbf(expf(rbf(S[(int64_t)(h * G + g) * s_stride + j] - M[g]))) : 0.f;
  }
  __syncthreads();
  if (wave < G) {
    const float s = wave_sum(p[wave][lane]);
    if (lane == 0) part_sum[split * heads + h * G + wave] = s;
  }
  {
    const int ch = tid % kLpp, jo = tid / kLpp;
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    bool page_ok = true;
    for (int jj = jo; jj < kSplit; jj += kGroups) {
      const int j = j0 + jj;
      if (j < jend) {
        bool ok = true;
        const int64_t off = page_offset(page_table, j, kv_heads, h, D, num_pages, &ok);
        if (!ok) {
          page_ok = false;
          continue;
        }
        const u32x4 vv = load16(vpool + off + ch * 8);
        const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float pj = p[g][jj];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            acc[g][2 * e] += rbf(pj * bf_lo(vw[e]));
            acc[g][2 * e + 1] += rbf(pj * bf_hi(vw[e]));
          }
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
  for (int o = tid; o < G * D; o += kBlock) {
    float s = 0.f;
    for (int q = 0; q < kGroups; ++q) s += red[q][o];
    part_out[((int64_t)split * heads + h * G) * D + o] = s;
  }
  // ---- last block of this kv head merges the splits
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int ticket = atomicAdd(&counters[h], 1);
    is_last = (ticket == participants - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const bf16* vnew = qkv + (int64_t)heads * D + (int64_t)kv_heads * D + h * D;
  for (int o = tid; o < G * D; o += kBlock) {
    const int g = o / D, d = o % D;
    float sp = 0.f, sv = 0.f;
    for (int s = 0; s < nact; ++s) {
      sp += part_sum[s * heads + h * G + g];
      sv += part_out[((int64_t)s * heads + h * G) * D + o];
    }
    const float pn = rbf(expf(rbf(snew[h * G + g] - M[g])));
    const float total = rbf(rbf(sp) + pn);
    const float weighted = rbf(rbf(sv) + rbf(pn * bf2f(vnew[d])));
    attn_out[(int64_t)(h * G + g) * D + d] = f2bf(weighted / total);
  }
  if (tid == 0) atomicExch(&counters[h], 0);
}

// ---------------------------------------------------------------------------
// host side: argument checks, error text, launches
// ---------------------------------------------------------------------------
thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
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

// error codes returned by the entries (negative; positive values are hipError_t)
enum : int { kBadArg = -1, kBadShape = -2, kUnsupported = -3 };

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

#define TFD_CMAX_SWITCH(K, CALL)                                          \
  switch (cmax_for(K)) {                                                  \
    case 1: { constexpr int kC = 1; CALL; break; }                        \
    case 2: { constexpr int kC = 2; CALL; break; }                        \
    case 4: { constexpr int kC = 4; CALL; break; }                        \
    case 8: { constexpr int kC = 8; CALL; break; }                        \
    case 12: { constexpr int kC = 12; CALL; break; }                      \
    case 16: { constexpr int kC = 16; CALL; break; }                      \
    default: return fail(kUnsupported, "K=%d exceeds 8192", K);           \
  }

template <int kC, int kR, int kPro, int kEpi>
void launch_gemv(const bf16* x, const bf16* gamma, const bf16* W, const bf16* resid, bf16* out,
                 int K, int N, float eps, hipStream_t s) {
  const int rows_per_block = kWavesPerBlock * kR;
  const int grid = (N + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((k_gemv<kC, kR, kPro, kEpi>), dim3(grid), dim3(kBlock), 0, s, x, gamma, W,
                     resid, out, K, N, eps);
}

}  // namespace

#include "../../include/tf_decode.h"

extern "C" {

const char* tfd_last_error(void) { return g_err; }

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
  else if (D == 128 && G == 4) { constexpr int kD = 128, kG = 4; CALL; }   \
  else if (D == 64 && G == 4) { constexpr int kD = 64, kG = 4; CALL; }     \
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

}  // extern "C"
