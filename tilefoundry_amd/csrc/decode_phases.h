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

#include <type_traits>

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
// The persistent kernel's GEMV: x is a bf16 vector in LDS (staged from
// flag-in-data words, or the embedding row), the residual too, and the output
// goes out as flag-in-data bf16 pairs.  Same arithmetic as gemv_finish.
// ---------------------------------------------------------------------------
template <int kCmax>
__device__ __forceinline__ void x_from_lds(const uint32_t* xs, int nch, int lane,
                                           u32x4 (&xr)[kCmax]) {
#pragma unroll
  for (int i = 0; i < kCmax; ++i) {
    const int c = i * kWave + lane;
    const u32x4 v = *reinterpret_cast<const u32x4*>(xs + 4 * (c < nch ? c : nch - 1));
    xr[i] = c < nch ? v : u32x4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ uint32_t bf_pair(bf16 lo, bf16 hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

// ---------------------------------------------------------------------------
// The row sums of kR (8 or 16) rows at once: lane l holds a partial sum of every
// row, and exchanges halve the rows a lane carries at each step -- lanes l and
// l ^ 32 (a lane swap: lanes below 32 keep rows 0 .. kR/2 - 1, the others the
// rest), l ^ 16 (lane swap), then within 16 lanes by mirrors, each pairing a
// lane with one of the other half -- until every lane holds one row, which the
// rest of its group then completes.  kR 16: lane l ends with row l / 4; kR 8:
// row l / 8; kR 4: row l / 16; every lane of a row's group holds the same bits.  About 35 VALU
// operations for 16 rows against 16 wave sums of 12.  (A row's f32 sum is taken
// in another order than wave_sum's.)
// ---------------------------------------------------------------------------
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xF, 0xF, false);
}
constexpr int kDppRor8 = 0x128;       // lane i <-> i + 8 (mod 16) within 16

template <int kR>
__device__ __forceinline__ float rows_sum(const float (&a)[kR], int lane) {
  static_assert(kR == 4 || kR == 8 || kR == 16, "4, 8 or 16 rows");
  constexpr int kH = kR / 2, kQ = kR / 4;
  float b[kH];
#pragma unroll
  for (int j = 0; j < kH; ++j) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[j]),
                                                    __float_as_uint(a[j + kH]), false, false);
    b[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  float c[kQ];
#pragma unroll
  for (int j = 0; j < kQ; ++j) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(b[j]),
                                                    __float_as_uint(b[j + kQ]), false, false);
    c[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  // within 16 lanes: lanes with bit 3 set keep the upper value of each pair;
  // the mirror (i <-> 15 - i) pairs every lane with one across bit 3
  const bool b3 = lane & 8;
  if constexpr (kR == 4) {
    return group_sum<16>(c[0]);
  } else if constexpr (kR == 8) {
    const float keep = b3 ? c[1] : c[0], give = b3 ? c[0] : c[1];
    float v = keep + dpp_f<kDppMirror>(give);
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppHalfMirror>(v);
    return v;
  } else {
    float d[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float keep = b3 ? c[k + 2] : c[k], give = b3 ? c[k] : c[k + 2];
      d[k] = keep + dpp_f<kDppMirror>(give);
    }
    const bool b2 = lane & 4;
    const float keep = b2 ? d[1] : d[0], give = b2 ? d[0] : d[1];
    float v = keep + dpp_f<kDppHalfMirror>(give);        // i <-> 7 - i: across bit 2
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppXor1>(v);
    return v;
  }
}

// The SwiGLU epilogue on rows_sum's layout (rows are (gate_n, up_n) pairs,
// model.py:230-233): every lane of a gate row's group takes the up row's sum
// from the next group, one silu for all pairs at once, and the pairs' words go
// out from one lane per word in one store.
template <int kR, int kPol>
__device__ __forceinline__ void swiglu_rows_out(const float (&part)[kR], int64_t row0,
                                                int nvalid, uint32_t* out, uint32_t tag,
                                                int lane) {
  const float y = rbf(rows_sum<kR>(part, lane));
  // the up row sits across bit 2 (16 rows) or bit 3 (8 rows) of the lane
  const float u = kR == 16 ? dpp_f<kDppHalfMirror>(y) : __uint_as_float(dpp_u<kDppRor8>(
                                                            __float_as_uint(y)));
  const uint32_t o = (uint32_t)f2bf(rbf(silu_f(y)) * u);
  // word q = (pair 2q, pair 2q + 1): 16 rows -- lanes 16q and 16q + 8; 8 rows
  // -- lanes 32q and 32q + 16
  uint32_t hi;
  if constexpr (kR == 16) {
    hi = dpp_u<kDppRor8>(o);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(o, o, false, false);
    hi = r[1];
  }
  constexpr int kLanesPerWord = kWave / (kR / 4);
  const int q = lane / kLanesPerWord;
  if (lane % kLanesPerWord == 0 && 4 * q + 3 < nvalid)
    ll_put<kPol>(out, (uint32_t)(row0 / 4 + q), (o & 0xffffu) | (hi << 16), tag);
}

// nbuf: the norm is shared by the block's waves through this LDS buffer
// (rms_norm_apply_block); then every wave of the block must call this with
// rows of its own (the caller's partition guarantees it).
template <int kCmax, int kR, int kPro, int kEpi, int kPol = kCoherent>
__device__ __forceinline__ void gemv_finish_ll(int vb, const uint32_t* xs,
                                               const u32x4 (&gr)[kCmax],
                                               const uint32_t* resid_s, uint32_t* out,
                                               uint32_t tag, int K, int N, float eps,
                                               const u32x4 (&w)[kR][kCmax],
                                               uint32_t* nbuf = nullptr) {
  static_assert(kR % 2 == 0, "outputs leave in pairs");
  static_assert(kEpi != kSwiglu || kR % 4 == 0, "swiglu outputs leave in pairs");
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row0 = ((int64_t)vb * kWavesPerBlock + wave) * kR;
  // a wave without rows still takes its part in a shared norm (block barrier)
  if (row0 >= N && !(kPro == kNorm && nbuf)) return;
  const int nvalid = (int)((N - row0) < kR ? (N - row0) : kR);
  u32x4 xr[kCmax];
  x_from_lds<kCmax>(xs, K / 8, lane, xr);
  if constexpr (kPro == kNorm && kCmax == kWavesPerBlock) {
    if (nbuf) rms_norm_apply_block<kCmax>(xr, gr, K, eps, nbuf);
    else rms_norm_apply<kCmax>(xr, gr, K, eps);
  } else if (kPro == kNorm) {
    rms_norm_apply<kCmax>(xr, gr, K, eps);
  }
  if (row0 >= N) return;
  if constexpr (kEpi == kSwiglu && (kR == 8 || kR == 16)) {
    float part[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < kCmax; ++i) a = dot8(w[r][i], xr[i], a);
      part[r] = a;
    }
    swiglu_rows_out<kR, kPol>(part, row0, nvalid, out, tag, lane);
    return;
  } else if constexpr ((kEpi == kStore || kEpi == kResid) && (kR == 8 || kR == 16)) {
    float part[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < kCmax; ++i) a = dot8(w[r][i], xr[i], a);
      part[r] = a;
    }
    // rows_sum's layout: row 2q + 1 sits across bit 2 (16 rows) or bit 3 (8)
    // of row 2q's lanes; word q leaves from the first lane of row 2q
    const float y0 = rbf(rows_sum<kR>(part, lane));
    const float y1 = kR == 16 ? dpp_f<kDppHalfMirror>(y0)
                              : __uint_as_float(dpp_u<kDppRor8>(__float_as_uint(y0)));
    constexpr int kLanesPerWord = kWave / (kR / 2);
    const int q = lane / kLanesPerWord;
    if (lane % kLanesPerWord == 0 && 2 * q + 1 < nvalid) {
      uint32_t pr;
      if (kEpi == kResid) {
        const uint32_t r = resid_s[(row0 + 2 * q) / 2];
        pr = bf_pair(f2bf(bf_lo(r) + y0), f2bf(bf_hi(r) + y1));
      } else {
        pr = bf_pair(f2bf(y0), f2bf(y1));
      }
      ll_put<kPol>(out, (uint32_t)((row0 + 2 * q) / 2), pr, tag);
    }
    return;
  }
  float acc[kR];
  dot_loaded<kCmax, kR>(w, xr, acc);
  if (kEpi == kSwiglu) {
    // rows come as (gate_n, up_n) pairs: mlp(), model.py:230-233
#pragma unroll
    for (int q = 0; q < kR / 4; ++q) {
      if (lane == q && 4 * q + 3 < nvalid) {
        bf16 o[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float g = rbf(acc[4 * q + 2 * e]);
          const float u = rbf(acc[4 * q + 2 * e + 1]);
          o[e] = f2bf(rbf(silu_f(g)) * u);
        }
        ll_put<kPol>(out, (uint32_t)(row0 / 4 + q), bf_pair(o[0], o[1]), tag);
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < kR / 2; ++q) {
      if (lane == q && 2 * q + 1 < nvalid) {
        const float y0 = rbf(acc[2 * q]), y1 = rbf(acc[2 * q + 1]);
        uint32_t pr;
        if (kEpi == kResid) {
          const uint32_t r = resid_s[(row0 + 2 * q) / 2];
          pr = bf_pair(f2bf(bf_lo(r) + y0), f2bf(bf_hi(r) + y1));
        } else {
          pr = bf_pair(f2bf(y0), f2bf(y1));
        }
        ll_put<kPol>(out, (uint32_t)((row0 + 2 * q) / 2), pr, tag);
      }
    }
  }
}

// One GEMV phase of the persistent kernel.  The weights of the block's first
// virtual block and the norm scales (gr, this lane's chunks) are already in
// flight, issued before the wait for x; further virtual blocks issue and
// finish in turn.
template <int kCmax, int kR, int kPro, int kEpi, int kPol = kCoherent>
__device__ __forceinline__ void gemv_ll(const uint32_t* xs, const u32x4 (&gr)[kCmax],
                                        const bf16* W, const uint32_t* resid_s, uint32_t* out,
                                        uint32_t tag, int K, int N, float eps,
                                        u32x4 (&w)[kR][kCmax]) {
  const int rows_per_vb = kWavesPerBlock * kR;
  for (int vb = blockIdx.x; vb * rows_per_vb < N; vb += gridDim.x) {
    if (vb != (int)blockIdx.x) gemv_issue<kCmax, kR>(vb, W, K, N, w);
    gemv_finish_ll<kCmax, kR, kPro, kEpi, kPol>(vb, xs, gr, resid_s, out, tag, K, N, eps, w);
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
// The step's last node in the persistent kernel: every block reduces all block
// picks (flag-in-data (value, index) pairs) the way finalize_phase does and
// derives the next token itself; block 0 also records the pick and publishes
// the token and position for the host.  Returns the next token.
// ---------------------------------------------------------------------------
template <class Grp = BlockGrp>
__device__ __forceinline__ int finalize_ll(const uint32_t* best, int nb, uint32_t tag, int p,
                                           const int* __restrict__ inp,
                                           const int* __restrict__ plen, int nsteps, int vocab,
                                           int64_t* ids, int* pos, int* sam, int* err) {
  const int tid = Grp::tid();
  float b = kNegInf;
  int i = 0x7fffffff;
  for (int k = tid; k < nb; k += kBlock) {
    const u32x2 v = ll_get2(best, 2u * k, tag, err);
    const float bv = __uint_as_float(v.x);
    const int bi = (int)v.y;
    if (better(bv, bi, b, i)) {
      b = bv;
      i = bi;
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
  __shared__ float sv[kWavesPerBlock];
  __shared__ int si[kWavesPerBlock];
  __shared__ int next_s;
  const int lane = tid & 63, wave = tid >> 6;
  if (lane == 0) {
    sv[wave] = b;
    si[wave] = i;
  }
  Grp::sync();
  if (tid == 0) {
    float bb = sv[0];
    int ii = si[0];
    for (int w = 1; w < kWavesPerBlock; ++w)
      if (better(sv[w], si[w], bb, ii)) {
        bb = sv[w];
        ii = si[w];
      }
    if (ii < 0 || ii >= vocab) ii = 0;  // all-NaN row: no pick exists
    int next = ii;
    if (p < 0 || p >= nsteps) {
      if (blockIdx.x == 0) raise_error(err, kErrStepRange);
    } else {
      if (blockIdx.x == 0) sam[p] = ii;
      if (p + 1 < plen[0] && p + 1 < nsteps) next = inp[p + 1];
    }
    if (next < 0 || next >= vocab) {
      if (blockIdx.x == 0) raise_error(err, kErrTokenRange);
      next = 0;
    }
    if (blockIdx.x == 0) {
      coh_sti64(ids, next);
      coh_sti(pos, p + 1);
    }
    next_s = next;
  }
  Grp::sync();
  return next_s;
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
  // P.V pass: kLpp lanes per position (16-byte chunks of V), kGroups positions
  static constexpr int kLpp = D / 8;
  static constexpr int kGroups = kBlock / kLpp;
  static constexpr int kVPasses = kSplit / kGroups;
  static_assert(kVPasses * kGroups == kSplit, "split tiles the P.V pass");
  // scores pass: kKLanes lanes per position, kKDims dims each, read as
  // kKChunks loads of which load i of the position's lanes covers 128
  // contiguous bytes (whole cache lines); kKPasses passes of the block per tile
  static constexpr int kKLanes = 8;
  static constexpr int kKDims = D / kKLanes;
  static constexpr int kKChunks = kKDims / 8;
  static constexpr int kKPpw = kWave / kKLanes;             // positions per wave and pass
  static constexpr int kKPasses = kSplit / (kWavesPerBlock * kKPpw);
  static_assert(kKPasses * kWavesPerBlock * kKPpw == kSplit, "passes cover a tile");
};

template <int D>
struct KTile {
  int pg[AttnShape<D>::kKPasses];          // the wave's page in each pass
  u32x4 t[AttnShape<D>::kKPasses][AttnShape<D>::kKChunks];
};
template <int D>
struct VTile {
  int pg[AttnShape<D>::kVPasses];
  u32x4 t[AttnShape<D>::kVPasses];
};

// position a thread reads in each pass layout
template <int D, class Grp = BlockGrp>
__device__ __forceinline__ int k_pos(int j0, int p) {
  using A = AttnShape<D>;
  const int lane = Grp::tid() & (kWave - 1), wave = Grp::tid() / kWave;
  return j0 + (p * kWavesPerBlock + wave) * A::kKPpw + lane / A::kKLanes;
}
template <int D, class Grp = BlockGrp>
__device__ __forceinline__ int v_pos(int j0, int p) {
  using A = AttnShape<D>;
  return j0 + (int)Grp::tid() / A::kLpp + p * A::kGroups;
}

// A wave's positions in one pass lie in one page (16 positions per wave in
// the scores pass; 64 / kLpp divides the page in the P.V pass), so the
// page-table entry is wave-uniform: a scalar load, which does not queue behind
// the tile loads already in flight the way a vector load would.
__device__ __forceinline__ int wave_page(const int* page_table, int max_pages, int first_pos) {
  const int pi = __builtin_amdgcn_readfirstlane(first_pos / kPage);
  return page_table[pi < max_pages ? pi : max_pages - 1];
}

// K rows of the 64 positions from j0 (positions j < P are the ones used): in
// pass p, lane l of wave w reads position j0 + 8 (4 p + w) + l / 8, chunks
// (l % 8) and (l % 8) + 8 (16 dims each), so a load instruction covers whole
// 128-byte lines.  A tile that holds no prior position issues nothing.
// K/V rows are read once per step.  Launches of one phase see the rows earlier
// launches wrote without device-scope loads (kCoh = false: streaming loads);
// the persistent kernel reads rows written earlier in the same launch, so its
// loads are device-coherent.
#ifndef TFD_KV_STREAM_POLICY
#define TFD_KV_STREAM_POLICY 2
#endif
template <bool kCoh>
__device__ __forceinline__ u32x4 kv_ld16(const void* base, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rsrc(base), byte_off, 0,
                                               kCoh ? kCoherent : TFD_KV_STREAM_POLICY);
}

// The pages of a K tile's passes: they depend on the positions only, so a
// kernel that reads the same positions in every layer can look them up once.
template <int D, class Grp = BlockGrp>
__device__ __forceinline__ void k_tile_pages(int j0, const int* page_table, int max_pages,
                                             KTile<D>& kt) {
  using A = AttnShape<D>;
  static_assert(kPage % A::kKPpw == 0, "a wave's positions of a pass stay in one page");
  const int wave = __builtin_amdgcn_readfirstlane((int)Grp::tid() / kWave);
#pragma unroll
  for (int p = 0; p < A::kKPasses; ++p)
    kt.pg[p] = wave_page(page_table, max_pages, j0 + (p * kWavesPerBlock + wave) * A::kKPpw);
}

// The K tile's loads from the pages already in kt.pg.
template <int D, bool kCoh, class Grp = BlockGrp>
__device__ __forceinline__ void k_tile_load_pages(int j0, int h, const bf16* kpool, int num_pages,
                                                  int kv_heads, KTile<D>& kt) {
  using A = AttnShape<D>;
  const int lane = Grp::tid() & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)Grp::tid() / kWave);
#pragma unroll
  for (int p = 0; p < A::kKPasses; ++p) {
    const bool bad = kt.pg[p] < 0 || kt.pg[p] >= num_pages;
    const int j = j0 + (p * kWavesPerBlock + wave) * A::kKPpw + lane / A::kKLanes;
    const int64_t row = page_row(bad ? 0 : kt.pg[p], j, kv_heads, h, D) + (lane % A::kKLanes) * 8;
#pragma unroll
    for (int i = 0; i < A::kKChunks; ++i)
      kt.t[p][i] = kv_ld16<kCoh>(kpool, (uint32_t)(row + 64 * i) * 2u);
  }
}

// pages and loads (the caller knows the tile holds a position below P)
template <int D, bool kCoh, class Grp = BlockGrp>
__device__ __forceinline__ void k_tile_load_at(int j0, int h, const int* page_table,
                                               int max_pages, const bf16* kpool, int num_pages,
                                               int kv_heads, KTile<D>& kt) {
  k_tile_pages<D, Grp>(j0, page_table, max_pages, kt);
  k_tile_load_pages<D, kCoh, Grp>(j0, h, kpool, num_pages, kv_heads, kt);
}

template <int D, bool kCoh, class Grp = BlockGrp>
__device__ __forceinline__ void k_tile_issue_at(int j0, int h, int P, const int* page_table,
                                                int max_pages, const bf16* kpool, int num_pages,
                                                int kv_heads, KTile<D>& kt) {
  using A = AttnShape<D>;
#pragma unroll
  for (int p = 0; p < A::kKPasses; ++p) {
    kt.pg[p] = -1;
#pragma unroll
    for (int i = 0; i < A::kKChunks; ++i) kt.t[p][i] = u32x4{0u, 0u, 0u, 0u};
  }
  if (j0 < P)
    k_tile_load_at<D, kCoh, Grp>(j0, h, page_table, max_pages, kpool, num_pages, kv_heads, kt);
}

template <int D, class Grp = BlockGrp>
__device__ __forceinline__ void v_tile_pages(int j0, const int* page_table, int max_pages,
                                             VTile<D>& vt) {
  using A = AttnShape<D>;
  static_assert(kPage % (kWave / A::kLpp) == 0, "a wave's pass stays in one page");
  const int wave = __builtin_amdgcn_readfirstlane((int)Grp::tid() / kWave);
#pragma unroll
  for (int p = 0; p < A::kVPasses; ++p)
    vt.pg[p] = wave_page(page_table, max_pages, j0 + p * A::kGroups + wave * (kWave / A::kLpp));
}

template <int D, bool kCoh, class Grp = BlockGrp>
__device__ __forceinline__ void v_tile_load_pages(int j0, int h, const bf16* vpool, int num_pages,
                                                  int kv_heads, VTile<D>& vt) {
  using A = AttnShape<D>;
  const int ch = (int)Grp::tid() % A::kLpp;
#pragma unroll
  for (int p = 0; p < A::kVPasses; ++p) {
    const int j = v_pos<D, Grp>(j0, p);
    const bool bad = vt.pg[p] < 0 || vt.pg[p] >= num_pages;
    vt.t[p] = kv_ld16<kCoh>(vpool, (uint32_t)(page_row(bad ? 0 : vt.pg[p], j, kv_heads, h, D) +
                                         ch * 8) * 2u);
  }
}

template <int D, bool kCoh, class Grp = BlockGrp>
__device__ __forceinline__ void v_tile_load_at(int j0, int h, const int* page_table,
                                               int max_pages, const bf16* vpool, int num_pages,
                                               int kv_heads, VTile<D>& vt) {
  v_tile_pages<D, Grp>(j0, page_table, max_pages, vt);
  v_tile_load_pages<D, kCoh, Grp>(j0, h, vpool, num_pages, kv_heads, vt);
}

template <int D, bool kCoh, class Grp = BlockGrp>
__device__ __forceinline__ void v_tile_issue_at(int j0, int h, int P, const int* page_table,
                                                int max_pages, const bf16* vpool, int num_pages,
                                                int kv_heads, VTile<D>& vt) {
  using A = AttnShape<D>;
#pragma unroll
  for (int p = 0; p < A::kVPasses; ++p) {
    vt.pg[p] = -1;
    vt.t[p] = u32x4{0u, 0u, 0u, 0u};
  }
  if (j0 < P)
    v_tile_load_at<D, kCoh, Grp>(j0, h, page_table, max_pages, vpool, num_pages, kv_heads, vt);
}

// The first tile of split `split` of a one-tile-per-split partition.
template <int D, bool kCoh, class Grp = BlockGrp>
__device__ __forceinline__ void k_tile_issue(int split, int h, int P, const int* page_table,
                                             int max_pages, const bf16* kpool, int num_pages,
                                             int kv_heads, KTile<D>& kt) {
  k_tile_issue_at<D, kCoh, Grp>(split * kSplit, h, P, page_table, max_pages, kpool, num_pages,
                           kv_heads, kt);
}
template <int D, bool kCoh, class Grp = BlockGrp>
__device__ __forceinline__ void v_tile_issue(int split, int h, int P, const int* page_table,
                                             int max_pages, const bf16* vpool, int num_pages,
                                             int kv_heads, VTile<D>& vt) {
  v_tile_issue_at<D, kCoh, Grp>(split * kSplit, h, P, page_table, max_pages, vpool, num_pages,
                           kv_heads, vt);
}

// ---------------------------------------------------------------------------
// Where the attention phases exchange data.  Per-phase launches (kLL = false)
// use plain device-coherent buffers and the kernel boundary as the barrier.
// The persistent kernel (kLL = true) uses flag-in-data words tagged with the
// (step, layer): the QKV projection, split maxima, numerator sums and P.V
// partials are polled for, and the merged output is published the same way.
// ---------------------------------------------------------------------------
struct AttnLL {
  const uint32_t* qkv;  // the layer's QKV projection, bf16 pairs
  uint32_t* smax;       // [split][heads] split maxima (f32)
  uint32_t* psum;       // [split][heads] numerator sums (f32)
  uint32_t* pout;       // [split][heads][D] P.V partials (f32)
  uint32_t* attn;       // [heads * D] merged output, bf16 pairs
  uint32_t tag;
};

// The head slice one kv head's blocks work on, staged in LDS as bf16 pairs:
// the G query vectors, then the key, then the value (D values each).
template <int D, int G>
__device__ __forceinline__ int head_src(int idx, int h, int heads, int kv_heads) {
  if (idx < G * D) return h * G * D + idx;
  if (idx < (G + 1) * D) return heads * D + h * D + (idx - G * D);
  return heads * D + kv_heads * D + h * D + (idx - (G + 1) * D);
}

template <int D, int G, class Grp = BlockGrp>
__device__ __forceinline__ void stage_head(int h, int heads, int kv_heads,
                                           const bf16* __restrict__ qkv, uint32_t* hs) {
  for (int i = Grp::tid(); i < (G + 2) * D / 2; i += kBlock) {
    const int src = head_src<D, G>(2 * i, h, heads, kv_heads);
    hs[i] = (uint32_t)qkv[src] | ((uint32_t)qkv[src + 1] << 16);
  }
}

template <int D, int G, int kPol = kCoherent, class Grp = BlockGrp>
__device__ __forceinline__ void stage_head_ll(int h, int heads, int kv_heads, const AttnLL& ll,
                                              uint32_t* hs, int* err) {
  // pairs of words: every run (q group, k, v) starts at an even word
  for (int i = Grp::tid(); i < (G + 2) * D / 4; i += kBlock) {
    const int src = head_src<D, G>(4 * i, h, heads, kv_heads);
    const u32x2 v = ll_get2<kPol>(ll.qkv, (uint32_t)src / 2u, ll.tag, err);
    hs[2 * i] = v.x;
    hs[2 * i + 1] = v.y;
  }
}

__device__ __forceinline__ float hs_at(const uint32_t* hs, int idx) {
  const uint32_t w = hs[idx >> 1];
  return (idx & 1) ? bf_hi(w) : bf_lo(w);
}

// Per-lane operands of the q/k norm and RoPE -- this wave's gamma pair and the
// rope-table pair at rp -- and the page of the new position.  They depend only
// on the layer and the position, so a caller can load them before the QKV
// projection exists.  Indices are clamped; part 1 raises the range errors.
struct QKPre {
  bf16 g0, g1, c0, s0, c1, s1;
  int page_new;
};

template <int D, int G, class Grp = BlockGrp>
__device__ __forceinline__ QKPre qk_prefetch(int rp, int P, const bf16* __restrict__ gq,
                                             const bf16* __restrict__ gk,
                                             const bf16* __restrict__ cos_t,
                                             const bf16* __restrict__ sin_t, int rope_rows,
                                             const int* __restrict__ page_table, int max_pages) {
  constexpr int kHalf = D / 2;
  const int lane = Grp::tid() & (kWave - 1), wave = Grp::tid() / kWave;
  const int li = lane < kHalf ? lane : 0;
  const int64_t r = (int64_t)((rp >= 0 && rp < rope_rows) ? rp : 0) * D;
  const int pg = (P >= 0 && P < max_pages * kPage) ? P / kPage : 0;
  // through a global address-space pointer: the select below would otherwise
  // make these FLAT loads, which also count against the LDS counter, so the
  // next LDS read would wait for every vector load issued before them
  typedef const __attribute__((address_space(1))) bf16 g_bf16;
  const g_bf16* gam = (const g_bf16*)(wave < G ? gq : gk);
  return QKPre{gam[li],           gam[li + kHalf],           cos_t[r + li], sin_t[r + li],
               cos_t[r + li + kHalf], sin_t[r + li + kHalf], page_table[pg]};
}

// The layer-dependent part of QKPre (the q/k norm scales), for a kernel that
// keeps the position-dependent part across layers.
template <int D, int G, class Grp = BlockGrp>
__device__ __forceinline__ void qk_gammas(const bf16* __restrict__ gq, const bf16* __restrict__ gk,
                                          QKPre& pre) {
  constexpr int kHalf = D / 2;
  const int lane = Grp::tid() & (kWave - 1), wave = Grp::tid() / kWave;
  const int li = lane < kHalf ? lane : 0;
  typedef const __attribute__((address_space(1))) bf16 g_bf16;
  const g_bf16* gam = (const g_bf16*)(wave < G ? gq : gk);
  pre.g0 = gam[li];
  pre.g1 = gam[li + kHalf];
}

// ---------------------------------------------------------------------------
// Part 1 (model.py:172-198).  Each block rebuilds its kv head's group of query
// vectors and the new key from the staged head slice: per-head RMS, RoPE at
// rp, q_s = bf16(q_rope * scale).  Split 0 writes this token's key and value
// into the paged cache at position P; every block scores the new key (the same
// bits in every block) and its own positions of the prior context,
//   s_j = bf16( sum_d bf16(q_s[d] * K[j][d]) ),
// and records the split's max per query head.
//
// A split is `chunks` tiles of 64 positions.  Per-phase launches keep the
// scores in global rows of s_stride; the flag-in-data kernels keep a block's
// own scores in LDS, G rows of chunks * 64.  `kt` holds the split's first tile
// (loaded by the caller); with kt1 (and kt2) the caller has also loaded the
// second (and third), so a split of up to that many tiles waits on no load
// issued inside this phase.
//
// kExact: the products of q_s and K are not rounded one by one; they are taken
// exactly (bf16 x bf16 fits f32) and summed in f32, as a matrix-core product
// does (the reference's fast path computes both attention products with
// T.gemm, examples/qwen3_1_7b-tilelang/fast/kernels.py:418-501).  Every other
// rounding point stays.  A pair of products is then one bf16 dot instruction
// on the cache word as loaded, where the rounded form takes five.
// ---------------------------------------------------------------------------
template <int D, int G, bool kLL, int kPol = kCoherent, class Grp = BlockGrp, bool kExact = false>
__device__ __forceinline__ void attn_scores_phase(
    int split, int h, const uint32_t* hs, const QKPre& pre, int rope_rows, int rp, int P,
    const int* __restrict__ page_table, int max_pages, bf16* __restrict__ kpool, bf16* __restrict__ vpool, int num_pages,
    int kv_heads, float scale, float eps, float* __restrict__ S, int s_stride,
    float* __restrict__ smax, float* __restrict__ snew, const AttnLL& ll, const KTile<D>& kt,
    int* err, int chunks = 1, const KTile<D>* kt1 = nullptr, const KTile<D>* kt2 = nullptr) {
  using A = AttnShape<D>;
  constexpr int kHalf = D / 2;
  static_assert(kHalf <= kWave, "one wave holds a head as (d, d + D/2) lane pairs");
  static_assert(G + 1 <= kWavesPerBlock, "one wave per vector");
  const int heads = kv_heads * G;
  const int tid = Grp::tid(), lane = tid & (kWave - 1), wave = tid / kWave;
  // a split is `chunks` tiles of 64 positions (the persistent kernel uses one)
  const int j0 = split * chunks * kSplit;

  // per-phase launches hand scores, maxima and new-key scores to the next
  // kernel, so plain (cached, write-back) stores are enough there
  auto put_max = [&](int g, float m) {
    if (kLL)
      ll_put<kPol>(ll.smax, (uint32_t)(split * heads + h * G + g), __float_as_uint(m), ll.tag);
    else
      smax[split * heads + h * G + g] = m;
  };
  if (split != 0 && j0 >= P) {
    if (tid < G) put_max(tid, kNegInf);
    return;
  }
  if (P < 0 || P >= max_pages * kPage || rp < 0 || rp >= rope_rows) {
    if (tid == 0) raise_error(err, kErrPosRange);
    if (tid < G) {
      put_max(tid, kNegInf);
      if (kLL)
        snew[tid] = 0.f;
      else
        snew[h * G + tid] = 0.f;
    }
    return;
  }
  // ---- the head slice is in LDS; gammas and rope rows came with `pre`
  const int v = wave;                     // vector this wave normalises (G queries + 1 key)
  const bool has_vec = v < G + 1;
  const bool isq = v < G;
  const bool act = has_vec && lane < kHalf;
  const int li = lane < kHalf ? lane : 0;
  const int vbase = (v < G + 1 ? v : 0) * D;
  const int page_new = pre.page_new;
  const int jend = (j0 + chunks * kSplit < P) ? j0 + chunks * kSplit : P;
  const float x0 = act ? hs_at(hs, vbase + li) : 0.f;
  const float x1 = act ? hs_at(hs, vbase + li + kHalf) : 0.f;
  const float g0 = bf2f(pre.g0), g1 = bf2f(pre.g1);
  const float c0 = bf2f(pre.c0), s0 = bf2f(pre.s0), c1 = bf2f(pre.c1), s1 = bf2f(pre.s1);

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
  Grp::sync();

  if (split == 0) {
    // this token's entry goes to the cache at P (fast/kernels.py:385-409)
    if (page_new < 0 || page_new >= num_pages) {
      if (tid == 0) raise_error(err, kErrPageRange);
    } else {
      const int64_t off = page_row(page_new, P, kv_heads, h, D);
      for (int d = tid; d < D; d += kBlock) {
        coh_st_bf16(kpool, (uint32_t)(off + d), f2bf(kn[d]));
        const uint32_t w = hs[((G + 1) * D + d) >> 1];
        coh_st_bf16(vpool, (uint32_t)(off + d), (bf16)((d & 1) ? (w >> 16) : (w & 0xffffu)));
      }
      // (later steps read these rows; in the persistent kernel the wait for
      // this block's next poll retires them before it publishes anything else)
    }
  }
  // score of the new key (score_new, model.py:198): per-phase launches keep
  // split 0's; the persistent kernel keeps every block's own copy in LDS
  if (wave < G) {
    float a = 0.f;
    if (lane < kHalf) {
      if (kExact) {
        a = qs[wave][lane] * kn[lane];
        a += qs[wave][lane + kHalf] * kn[lane + kHalf];
      } else {
        a = rbf(qs[wave][lane] * kn[lane]);
        a += rbf(qs[wave][lane + kHalf] * kn[lane + kHalf]);
      }
    }
    a = wave_sum(a);
    if (lane == 0) {
      if (kLL)
        snew[wave] = rbf(a);
      else if (split == 0)
        snew[h * G + wave] = rbf(a);
    }
  }

  // ---- scores over this split of the prior context: kKLanes lanes per
  // position; lane part p holds dims 8 (8 i + p) .. +7 of chunk i
  constexpr int kKL = A::kKLanes;
  const int part = lane % kKL;
  float qv[G][A::kKChunks][8];
  uint32_t qp[G][A::kKChunks][4];          // kExact: the same dims as bf16 pairs
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < A::kKChunks; ++i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[g][i][e] = qs[g][8 * (kKL * i + part) + e];
#pragma unroll
      for (int e = 0; e < 4; ++e) qp[g][i][e] = pack2(qv[g][i][2 * e], qv[g][i][2 * e + 1]);
    }
  float mymax[G];
#pragma unroll
  for (int g = 0; g < G; ++g) mymax[g] = kNegInf;
  bool page_ok = true;
  // tile c is reduced from `cur` while tile c + 1 loads into `nxt`; the two
  // buffers alternate (no copy between them), and every tile but the last
  // issues the next one's loads unconditionally, so the wait for `cur` never
  // has to cover a path without them (which would make it wait for `nxt`)
  const int ntl = (jend - j0 + kSplit - 1) / kSplit;    // tiles with a position < jend
  auto tile = [&](int c, const KTile<D>& cur, KTile<D>& nxt, auto issue) {
    const int jc = j0 + c * kSplit;
    if (decltype(issue)::value)
      k_tile_load_at<D, kLL, Grp>(jc + kSplit, h, page_table, max_pages, kpool, num_pages, kv_heads,
                             nxt);
#pragma unroll
    for (int p = 0; p < A::kKPasses; ++p) {
      const int j = k_pos<D, Grp>(jc, p);
      const bool bad = cur.pg[p] < 0 || cur.pg[p] >= num_pages;
      if (j < jend && bad) page_ok = false;
      const bool valid = j < jend && !bad;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < A::kKChunks; ++i) {
          const uint32_t kw[4] = {cur.t[p][i].x, cur.t[p][i].y, cur.t[p][i].z, cur.t[p][i].w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            a = kExact ? dot2(qp[g][i][e], kw[e], a)
                       : add_rounded2(a, qv[g][i][2 * e] * bf_lo(kw[e]),
                                      qv[g][i][2 * e + 1] * bf_hi(kw[e]));
        }
        a = group_sum<kKL>(a);
        const float sc = rbf(a);
        if (valid) {
          if (part == 0) {
            if (kLL)
              S[g * chunks * kSplit + (j - j0)] = sc;
            else
              S[(int64_t)(h * G + g) * s_stride + j] = sc;
          }
          mymax[g] = fmaxf(mymax[g], sc);
        }
      }
    }
  };
  // tiles c, c + 1, ... from `cur`, the buffers alternating
  auto run = [&](int c, KTile<D>& cur, KTile<D>& oth) {
    for (; c + 2 < ntl; c += 2) {
      tile(c, cur, oth, std::true_type{});
      tile(c + 1, oth, cur, std::true_type{});
    }
    if (c + 1 < ntl) {
      tile(c, cur, oth, std::true_type{});
      tile(c + 1, oth, cur, std::false_type{});
    } else if (c < ntl) {
      tile(c, cur, oth, std::false_type{});
    }
  };
  KTile<D> ka = kt, kb;
  if (kt1 != nullptr && ntl >= 2) {
    // tile 1 (and 2) came with the caller's loads; later tiles load in turn
    kb = *kt1;
    tile(0, ka, kb, std::false_type{});
    if (kt2 != nullptr && ntl >= 3) {
      ka = *kt2;
      tile(1, kb, ka, std::false_type{});
      run(2, ka, kb);
    } else {
      run(1, kb, ka);
    }
  } else {
    run(0, ka, kb);
  }
  if (!page_ok) raise_error(err, kErrPageRange);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = wave_max(mymax[g]);
    if (lane == 0) wmax[wave][g] = m;
  }
  Grp::sync();
  if (tid < G) {
    float m = wmax[0][tid];
    for (int w = 1; w < kWavesPerBlock; ++w) m = fmaxf(m, wmax[w][tid]);
    put_max(tid, m);
  }
  Grp::sync();
}

__device__ __forceinline__ float sn_of(const float* snew, int i) { return coh_ldf(&snew[i]); }

// The last step of the softmax for one output (model.py:206-212): with the
// joint peak M, the split sums in split order sp and sv, and the new key's
// score and value,
//   total    = bf16(bf16(sp) + p_new),  p_new = bf16(exp(bf16(s_new - M)))
//   weighted = bf16(bf16(sv) + bf16(p_new * v_new))
//   out      = bf16(weighted / total)
__device__ __forceinline__ bf16 attn_merge_one(float sp, float sv, float sn, float M,
                                               float vnew) {
  const float pn = rbf(expf(rbf(sn - M)));
  const float total = rbf(rbf(sp) + pn);
  const float weighted = rbf(rbf(sv) + rbf(pn * vnew));
  return f2bf(weighted / total);
}

// ---------------------------------------------------------------------------
// Part 2 (model.py:200-212).  With the joint peak M = max(split maxima, score_new):
//   p_j = bf16(exp(bf16(s_j - M)))
//   per split: sum_j p_j and sum_j bf16(p_j * V[j][d]) in f32
// Per-phase launches merge in the last block of a kv head to finish (a per-head
// counter decides; partials go through device-coherent stores, and each wave
// waits for its own before the block counts itself in), staging the partials
// through LDS with coalesced loads and summing in split order.  The persistent
// kernel publishes the partials as flag-in-data words and merges in part 3.
// ---------------------------------------------------------------------------
struct NoHook {
  __device__ void operator()() const {}
};
// Where output value k of the attention row goes (element index from attn_out).
struct RowOut {
  __device__ uint32_t operator()(int k) const { return (uint32_t)k; }
};

// `polled` runs once this block's waits of the phase are over (the persistent
// kernel issues weight loads there: memory counters retire in order, so loads
// issued before a wait would hold it up)
//
// kExact: sum_j p_j * V[j][d] with the products exact and summed in f32 (no
// per-product rounding; see attn_scores_phase): the two positions of a pass
// pair meet in one bf16 dot instruction, their p_j and their V entries each
// packed as a pair by one byte permute.
template <int D, int G, bool kLL, class Hook = NoHook, class OutMap = RowOut,
          int kPol = kCoherent, class Grp = BlockGrp, bool kExact = false>
__device__ __forceinline__ void attn_pv_phase(
    int split, int h, int nsplit, const bf16* __restrict__ qkv, int P,
    const int* __restrict__ page_table, int max_pages, const bf16* __restrict__ vpool,
    int num_pages, int kv_heads, const float* __restrict__ S, int s_stride,
    const float* __restrict__ smax, const float* __restrict__ snew, float* part_sum,
    float* part_out, int* counters, bf16* __restrict__ attn_out, const AttnLL& ll,
    const VTile<D>& vt, int* err, int chunks = 1, const Hook& polled = Hook(),
    const OutMap& omap = OutMap(), const VTile<D>* vt1 = nullptr,
    const VTile<D>* vt2 = nullptr) {
  using A = AttnShape<D>;
  constexpr int kLpp = A::kLpp;
  constexpr int kGroups = A::kGroups;
  constexpr int kOut = G * D;                         // outputs of the head group
  static_assert(kSplit == kWave, "one wave sums one head's tile of p");
  static_assert(G <= kWavesPerBlock, "one wave per query head of the group");
  static_assert(kOut % 4 == 0 && kOut <= kBlock, "one thread per output");
  const int heads = kv_heads * G;
  const int tid = Grp::tid(), lane = tid & (kWave - 1), wave = tid / kWave;
  const int ch = tid % kLpp, jo = tid / kLpp;
  // a split is `chunks` tiles of 64 positions (the persistent kernel uses one)
  const int slen = chunks * kSplit;
  const int j0 = split * slen;

  if (P < 0 || P >= max_pages * kPage) P = 0;  // part 1 already raised the flag
  const int nact = (P + slen - 1) / slen;
  const int participants = nact > 0 ? nact : 1;
  if (split >= participants) return;
  const int jend = (j0 + slen < P) ? j0 + slen : P;

  // ---- the first tile's scores, every split's max, the new-key scores
  const int wg = wave < G ? wave : 0;
  // the persistent kernel passes this block's own scores and new-key scores (LDS)
  const float sn = kLL ? snew[wg] : snew[h * G + wg];
  // flag-in-data kernels: this block's scores in LDS, G rows of slen
  const float sj_first =
      kLL ? S[wg * slen + lane] : S[(int64_t)(h * G + wg) * s_stride + j0 + lane];
  float mx = kNegInf;
  for (int s0 = 0; s0 < nact; s0 += kWave) {
    const int s = s0 + lane;
    float m;
    if (kLL) {
      // lanes past the active splits re-read split 0's word (always written)
      m = __uint_as_float(
          ll_get<kPol>(ll.smax, (uint32_t)((s < nact ? s : 0) * heads + h * G + wg), ll.tag, err));
    } else {
      m = smax[(s < nsplit ? s : nsplit - 1) * heads + h * G + wg];
    }
    if (s < nact) mx = fmaxf(mx, m);
  }
  polled();

  __shared__ float M[G];
  __shared__ float p[G][kSplit];
  __shared__ float red[kGroups][kOut];
  __shared__ float psums[kGroups][G];
  __shared__ int is_last;

  float mw = 0.f;                                     // wave g's joint peak
  if (wave < G) {
    mw = fmaxf(wave_max(mx), sn);
    if (lane == 0) M[wave] = mw;
  }
  float psum = 0.f;                                   // wave g: sum of p, tile by tile
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  bool page_ok = true;
  // have the first scores here, on every path, so no wait for them is left
  // pending into the tile loop (where it would also wait for the V rows the
  // loop prefetches)
  asm volatile("" ::"v"(sj_first));
  // tile c is reduced from `cur` (scores sj) while tile c + 1's scores, then
  // its V rows, load into `nxt` / sj_next -- the scores first: memory counters
  // retire in order, so waiting for them does not wait for the V rows.  The
  // buffers alternate (no copy between them), and every tile but the last
  // issues the next one's loads unconditionally.
  const int ntl = (jend - j0 + kSplit - 1) / kSplit;    // tiles with a position < jend
  auto tile = [&](int c, const VTile<D>& cur, float sj, VTile<D>& nxt, float& sj_next,
                  auto issue) {
    const int jc = j0 + c * kSplit;
    if (kLL && c > 0) sj = S[wg * slen + (jc - j0) + lane];   // LDS: no prefetch needed
    if (decltype(issue)::value) {
      if (!kLL) {
        // lanes past jend read a score of this row (in bounds, unused)
        const int jn = jc + kSplit + lane;
        sj_next = S[(int64_t)(h * G + wg) * s_stride + (jn < jend ? jn : jend - 1)];
      }
      v_tile_load_at<D, kLL, Grp>(jc + kSplit, h, page_table, max_pages, vpool, num_pages, kv_heads,
                             nxt);
    }
    if (wave < G) {
      const float pj = (jc + lane < jend) ? rbf(expf(rbf(sj - mw))) : 0.f;
      p[wave][lane] = pj;
      psum += wave_sum(pj);
    }
    Grp::sync();
    // passes q and q + 1 hold the same dims of two positions: their rounded
    // products go to each accumulator as one pair
    static_assert(A::kVPasses % 2 == 0, "passes pair up");
#pragma unroll
    for (int q = 0; q < A::kVPasses; q += 2) {
      uint32_t vw[2][4];
      float pj[2][G];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int jj = jo + (q + u) * kGroups;
        const bool bad = cur.pg[q + u] < 0 || cur.pg[q + u] >= num_pages;
        if (jc + jj < jend && bad) page_ok = false;
        const u32x4 t = (jc + jj < jend && !bad) ? cur.t[q + u] : u32x4{0u, 0u, 0u, 0u};
        vw[u][0] = t.x;
        vw[u][1] = t.y;
        vw[u][2] = t.z;
        vw[u][3] = t.w;
#pragma unroll
        for (int g = 0; g < G; ++g) pj[u][g] = p[g][jj];   // 0 past the end: exact zeros
      }
      if constexpr (kExact) {
        // (V[j0][d], V[j1][d]) and (V[j0][d+1], V[j1][d+1]) from the two words;
        // (p_j0, p_j1) from the high halves of the two bf16-valued floats
        uint32_t vl[4], vh[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vl[e] = __builtin_amdgcn_perm(vw[1][e], vw[0][e], 0x05040100u);
          vh[e] = __builtin_amdgcn_perm(vw[1][e], vw[0][e], 0x07060302u);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const uint32_t pp = __builtin_amdgcn_perm(__float_as_uint(pj[1][g]),
                                                    __float_as_uint(pj[0][g]), 0x07060302u);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            acc[g][2 * e] = dot2(pp, vl[e], acc[g][2 * e]);
            acc[g][2 * e + 1] = dot2(pp, vh[e], acc[g][2 * e + 1]);
          }
        }
      } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            acc[g][2 * e] = add_rounded2(acc[g][2 * e], pj[0][g] * bf_lo(vw[0][e]),
                                         pj[1][g] * bf_lo(vw[1][e]));
            acc[g][2 * e + 1] = add_rounded2(acc[g][2 * e + 1], pj[0][g] * bf_hi(vw[0][e]),
                                             pj[1][g] * bf_hi(vw[1][e]));
          }
        }
      }
    }
    Grp::sync();                        // p is rewritten by the next tile
  };
  // tiles c, c + 1, ... from `cur`, the buffers alternating
  auto run = [&](int c, VTile<D>& cur, float& scur, VTile<D>& oth, float& soth) {
    for (; c + 2 < ntl; c += 2) {
      tile(c, cur, scur, oth, soth, std::true_type{});
      tile(c + 1, oth, soth, cur, scur, std::true_type{});
    }
    if (c + 1 < ntl) {
      tile(c, cur, scur, oth, soth, std::true_type{});
      tile(c + 1, oth, soth, cur, scur, std::false_type{});
    } else if (c < ntl) {
      tile(c, cur, scur, oth, soth, std::false_type{});
    }
  };
  VTile<D> va = vt, vb;
  float sa = sj_first, sb = 0.f;
  if (kLL && vt1 != nullptr && ntl >= 2) {
    // tile 1 (and 2) came with the caller's loads; later tiles load in turn
    // (flag-in-data kernels read each tile's scores from LDS)
    vb = *vt1;
    tile(0, va, sa, vb, sb, std::false_type{});
    if (vt2 != nullptr && ntl >= 3) {
      va = *vt2;
      tile(1, vb, sb, va, sa, std::false_type{});
      run(2, va, sa, vb, sb);
    } else {
      run(1, vb, sb, va, sa);
    }
  } else {
    run(0, va, sa, vb, sb);
  }
  if (!page_ok) raise_error(err, kErrPageRange);
  if (wave < G && lane == 0) {
    if (kLL)
      ll_put<kPol>(ll.psum, (uint32_t)(split * heads + h * G + wave), __float_as_uint(psum), ll.tag);
    else
      coh_stf(&part_sum[split * heads + h * G + wave], psum);
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[jo][g * D + ch * 8 + e] = acc[g][e];
  Grp::sync();
  if (kLL) {
    for (int o = 2 * tid; o < kOut; o += 2 * kBlock) {
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int q = 0; q < kGroups; ++q) {
        s0 += red[q][o];
        s1 += red[q][o + 1];
      }
      ll_put2<kPol>(ll.pout, (uint32_t)(((int64_t)split * heads + h * G) * D + o), __float_as_uint(s0),
              __float_as_uint(s1), ll.tag);
    }
    Grp::sync();
    return;
  }
  for (int o = tid; o < kOut; o += kBlock) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < kGroups; ++q) s += red[q][o];
    coh_stf(&part_out[((int64_t)split * heads + h * G) * D + o], s);
  }
  // ---- the last block of this kv head merges the splits
  stores_done();
  Grp::sync();
  if (tid == 0) {
    const int ticket = atomicAdd(&counters[h], 1);
    is_last = (ticket == participants - 1);
  }
  Grp::sync();
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
    Grp::sync();
    if (tid < kOut) {
      for (int s = 0; s < nc; ++s) {
        sv += red[s][tid];
        sp += psums[s][tid / D];
      }
    }
    Grp::sync();
  }
  if (tid < kOut) {
    const int g = tid / D, d = tid % D;
    const uint32_t vnew = (uint32_t)(heads * D + kv_heads * D + h * D);
    coh_st_bf16(attn_out, omap((h * G + g) * D + d),
                attn_merge_one(sp, sv, sn_of(snew, h * G + g), M[g], bf2f(qkv[vnew + d])));
  }
  if (tid == 0) atomicExch(&counters[h], 0);
  Grp::sync();
}

// ---------------------------------------------------------------------------
// Part 3, persistent kernel only: every active split of a kv head merges its
// own slice of the head group's G * D outputs (pairs of values), reading every
// split's partials for that slice and the numerator sums, in split order --
// the same arithmetic as the last-block merge above.  Up to kChunk splits at a
// time, every word of a chunk (partial sums, maxima, partial outputs and the
// new key's values) polled in one round: a thread holds at most one of each.
// Splits are `chunks` tiles of 64 positions, as in parts 1 and 2.
// ---------------------------------------------------------------------------
template <int D, int G, class Hook = NoHook, int kPol = kCoherent, class Grp = BlockGrp>
__device__ __forceinline__ void attn_merge_ll(int split, int h, int P, int max_pages,
                                              int kv_heads, const float* snew, const AttnLL& ll,
                                              int* err, const Hook& polled = Hook(),
                                              int chunks = 1) {
  constexpr int kPairs = G * D / 2;
  constexpr int kChunk = 32;                          // splits staged at a time
  static_assert(kChunk * G <= kBlock && kPairs + kChunk <= kBlock, "one word of a kind per thread");
  const int heads = kv_heads * G;
  const int tid = Grp::tid();
  if (P < 0 || P >= max_pages * kPage) P = 0;
  const int nact = (P + chunks * kSplit - 1) / (chunks * kSplit);
  const int participants = nact > 0 ? nact : 1;
  if (split >= participants) return;
  const int q0 = split * kPairs / participants, q1 = (split + 1) * kPairs / participants;
  const int nq = q1 - q0;

  __shared__ float sm[kChunk][G], ps[kChunk][G];
  // a chunk's partial outputs, split-major: nc * nq <= kPairs + kChunk - 1
  __shared__ u32x2 po[kPairs + kChunk];
  float sv0 = 0.f, sv1 = 0.f, sp = 0.f, mx = kNegInf;
  const int o = 2 * (q0 + (tid < nq ? tid : 0));
  const int g = o / D, d = o % D;
  // the new key's values d, d + 1 (one word of the QKV projection)
  const uint32_t wv = (uint32_t)(heads * D + kv_heads * D + h * D + d) / 2u;
  uint32_t vw = 0;
  for (int c0 = 0; c0 < participants; c0 += kChunk) {
    const int nc = (participants - c0) < kChunk ? (participants - c0) : kChunk;
    const bool has_s = tid < nc * G;
    // split maxima exist only for splits holding a prior position
    const bool has_m = has_s && c0 + tid / G < nact;
    const bool has_o = tid < nc * nq;
    const bool has_v = c0 == 0 && tid < nq;
    const int is = has_s ? tid : 0, io = has_o ? tid : 0;
    const uint32_t ws = (uint32_t)((c0 + is / G) * heads + h * G + is % G);
    const uint32_t wo = (uint32_t)(((int64_t)(c0 + io / nq) * heads + h * G) * D + 2 * (q0 + io % nq));
    u32x2 a, b, v;
    u32x4 c;
    uint32_t spins = 0;
    for (;;) {
      a = __builtin_amdgcn_raw_buffer_load_b64(rsrc(ll.psum), ws * 8u, 0, ld_bits(kPol));
      b = __builtin_amdgcn_raw_buffer_load_b64(rsrc(ll.smax), ws * 8u, 0, ld_bits(kPol));
      c = __builtin_amdgcn_raw_buffer_load_b128(rsrc(ll.pout), wo * 8u, 0, ld_bits(kPol));
      v = __builtin_amdgcn_raw_buffer_load_b64(rsrc(ll.qkv), wv * 8u, 0, ld_bits(kPol));
      const bool ok = (!has_s || a.y == ll.tag) && (!has_m || b.y == ll.tag) &&
                      (!has_o || (c.y == ll.tag && c.w == ll.tag)) && (!has_v || v.y == ll.tag);
      if (ok || ll_give_up(spins, err)) break;
      __asm__ volatile("" ::: "memory");
    }
    if (has_s) {
      ps[is / G][is % G] = __uint_as_float(a.x);
      sm[is / G][is % G] = has_m ? __uint_as_float(b.x) : kNegInf;
    }
    if (has_o) po[io] = u32x2{c.x, c.z};
    if (has_v) vw = v.x;
    Grp::sync();
    if (c0 == 0) polled();
    if (tid < nq) {
      for (int s = 0; s < nc; ++s) {
        sv0 += __uint_as_float(po[s * nq + tid].x);
        sv1 += __uint_as_float(po[s * nq + tid].y);
        sp += ps[s][g];
        mx = fmaxf(mx, sm[s][g]);
      }
    }
    Grp::sync();
  }
  if (tid < nq) {
    const float sn = snew[g];
    const float M = fmaxf(mx, sn);
    const bf16 r0 = attn_merge_one(sp, sv0, sn, M, bf_lo(vw));
    const bf16 r1 = attn_merge_one(sp, sv1, sn, M, bf_hi(vw));
    ll_put<kPol>(ll.attn, (uint32_t)((h * G * D + o) / 2), (uint32_t)r0 | ((uint32_t)r1 << 16), ll.tag);
  }
}

}  // namespace tfd
