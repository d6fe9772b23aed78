// Device helpers shared by the hybrid models' kernels (hybrid.hip, the
// small-batch kernels of hybrid_small.hip, twin_ops.hip): operand-order
// offsets, activations, the routers, the experts' weight chunks and the
// f32 convolution step.
#pragma once

#include "decode_phases.h"

namespace tfd_hybrid {

using namespace tfd;

// the skinny GEMMs' operand order for a [rows <= 32][K] activation
__device__ __forceinline__ int64_t xp_off_h(int m, int k) {
  return ((int64_t)((k >> 5) * 2 + (m >> 4)) * 64 + (m & 15) + 16 * ((k >> 3) & 3)) * 8 +
         (k & 7);
}

__device__ __forceinline__ float softplus_f(float x) {
  // torch.nn.functional.softplus (beta 1, threshold 20)
  return x > 20.f ? x : log1pf(expf(x));
}
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }

// ---------------------------------------------------------------------------
// Routers: one wave per row of E <= 256 f32 logits.  The top k are taken by
// value, largest first, equal values by ascending index (torch.topk leaves the
// order of ties open; bf16-valued logits tie often).  Qwen3.5 ranks the softmax
// probabilities: softmax is increasing, so ranking the logits ranks them too,
// except that two logits closer than an f32 ulp of the largest one (both
// within 2^-24 of zero beside a logit of 1, say) round to one probability, and
// there the larger logit goes first.
//   kMode 0 (torch_ref.py:417-430): p = softmax over all E in f32, weights =
//            p_topk / sum p_topk (f32)
//   kMode 1 (granite model.py:376-390): weights = bf16(softmax over the top k)
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wave_min_i(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(0, v, kDppXor1, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, kDppXor2, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, kDppHalfMirror, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, kDppMirror, 0xF, 0xF, false));
  v = min(v, __shfl_xor(v, 16, kWave));
  const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return min((int)r[0], (int)r[1]);
}

// The k picks of one row, held by lanes 0..k-1 (lane r: the r-th pick's
// weight and expert id; other lanes' values are meaningless).
template <int kMode>
__device__ __forceinline__ void route_core(const float* __restrict__ lrow, int E, int k, int lane,
                                           float& weight, int& expert) {
  float v[4];
  int id[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + kWave * j;
    id[j] = e;
    v[j] = e < E ? lrow[e] : kNegInf;
  }
  const float m = wave_max(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
  float sum_all = 0.f;
  if (kMode == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (id[j] < E) sum_all += expf(v[j] - m);
    sum_all = wave_sum(sum_all);
  }
  bool taken[4] = {false, false, false, false};
  float my_val = kNegInf;
  int my_idx = 0;
  for (int r = 0; r < k; ++r) {
    // this lane's best candidate (ids grow with j, so ties keep the first)
    float bv = kNegInf;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (id[j] < E && !taken[j] && (bi == 0x7fffffff || v[j] > bv)) {
        bv = v[j];
        bi = id[j];
      }
    // the wave's largest value, then the lowest id holding it
    const float wm = wave_max(bv);
    int pick = wave_min_i(bi != 0x7fffffff && bv == wm ? bi : 0x7fffffff);
    if (pick == 0x7fffffff) pick = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (id[j] == pick) taken[j] = true;
    if (lane == r) {
      my_val = wm;
      my_idx = pick;
    }
  }
  // weights of the k picks, held by lanes 0..k-1
  float w = 0.f;
  if (lane < k) w = kMode == 0 ? expf(my_val - m) / sum_all : expf(my_val - m);
  const float tot = wave_sum(lane < k ? w : 0.f);
  weight = kMode == 0 ? w / tot : rbf(w / tot);
  expert = my_idx;
}

template <int kMode>
__device__ __forceinline__ void route_row(const float* __restrict__ lrow, int E, int k,
                                          float* __restrict__ wrow, int* __restrict__ irow,
                                          int lane) {
  float w;
  int e;
  route_core<kMode>(lrow, E, k, lane, w, e);
  if (lane < k) {
    wrow[lane] = w;
    irow[lane] = e;
  }
}

template <bool kFp8>
struct WChunk;
template <>
struct WChunk<false> {
  using T = u32x4;
  static __device__ __forceinline__ T load(const void* w, int64_t row, int K, int c) {
    return load16_stream((const bf16*)w + row * K + (int64_t)c * 8);
  }
  static __device__ __forceinline__ float dot(const T& w, const u32x4& x, float acc) {
    return dot8(w, x, acc);
  }
};
template <>
struct WChunk<true> {
  using T = u32x2;
  static __device__ __forceinline__ T load(const void* w, int64_t row, int K, int c) {
    return __builtin_nontemporal_load(
        reinterpret_cast<const u32x2*>((const uint8_t*)w + row * K + (int64_t)c * 8));
  }
  // e4m3fn values are exact in bf16: gfx950's scaled fp8 -> bf16 pair
  // conversion at scale 1.0 decodes every code exactly (bytes 0-1, then 2-3
  // with `sel`); then bf16 dot products
  static __device__ __forceinline__ float dot(const T& q, const u32x4& x, float acc) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    const bf16x2_v v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.x, 1.0f, false);
    const bf16x2_v v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.x, 1.0f, true);
    const bf16x2_v v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.y, 1.0f, false);
    const bf16x2_v v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.y, 1.0f, true);
    const u32x4 wv = {__builtin_bit_cast(uint32_t, v0), __builtin_bit_cast(uint32_t, v1),
                      __builtin_bit_cast(uint32_t, v2), __builtin_bit_cast(uint32_t, v3)};
    return dot8(wv, x, acc);
  }
};

// x's chunks c = lane + 64 i (zero past the end)
template <int kC>
__device__ __forceinline__ void load_vec(const bf16* x, int K, int lane, u32x4 (&xr)[kC]) {
  const int nch = K / 8;
#pragma unroll
  for (int i = 0; i < kC; ++i) {
    const int c = lane + kWave * i;
    xr[i] = c < nch ? load16(x + (int64_t)c * 8) : u32x4{0u, 0u, 0u, 0u};
  }
}

// a row of K weights against x, summed over the wave (every lane gets it)
template <bool kFp8, int kC>
__device__ __forceinline__ float row_dot(const void* w, int64_t row, int K, const u32x4 (&x)[kC],
                                         int lane) {
  float acc = 0.f;
  const int nch = K / 8;
#pragma unroll
  for (int i = 0; i < kC; ++i) {
    const int c = lane + kWave * i;
    if (c < nch) acc = WChunk<kFp8>::dot(WChunk<kFp8>::load(w, row, K, c), x[i], acc);
  }
  return wave_sum(acc);
}

template <int kD, int kKW>
__device__ __forceinline__ float conv_silu_f32(const float* cin, const bf16* w, float entry,
                                               float* cout, bool write) {
  float acc = 0.f;
  float win[kKW];
#pragma unroll
  for (int t = 0; t < kKW - 1; ++t) win[t] = cin[t];
  win[kKW - 1] = entry;
#pragma unroll
  for (int t = 0; t < kKW; ++t) acc += win[t] * bf2f(w[t]);
  if (write) {
#pragma unroll
    for (int t = 0; t < kKW - 1; ++t) cout[t] = win[t + 1];
  }
  return silu_f(acc);
}

}  // namespace tfd_hybrid
