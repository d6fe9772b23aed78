// Device-side building blocks shared by every decode kernel (gfx950, wave64).
//
// Numerics contract.  The authored Qwen3 HIR (examples/qwen3_1_7b-tilelang/
// ref_src/model.py:125-234) rounds to bf16 after every op it declares at bf16,
// and the reference evaluator computes each such op in f32 and rounds once
// (torch CPU semantics for bf16 tensors).  The helpers below reproduce that:
//   * rbf(x)   rounds an f32 to the nearest-even bf16 and back (c10::BFloat16's
//              rule, NaN -> 0x7fc0);
//   * the file is compiled with -ffp-contract=off so `a * b + c` stays two
//     rounded ops, as two torch ops are; FMAs are written out (fmaf) only in
//     dot-product accumulations, whose order is not the reference's anyway;
//   * reductions run in f32 in a fixed order (lane-sequential, then an xor
//     butterfly), so every block that recomputes a reduction gets the same bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tfd {

typedef uint16_t bf16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kBlock = 256;           // 4 waves
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kPage = 16;             // KV positions per page
constexpr int kSplit = 64;            // context positions per attention block

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(bf16 b) { return __uint_as_float(((uint32_t)b) << 16); }

__device__ __forceinline__ bf16 f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (bf16)0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16)(u >> 16);
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

// Sum over the 64 lanes; every lane ends with the same bits (a + b == b + a).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// Sum within aligned groups of `width` lanes (width a power of two <= 64).
template <int kWidth>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = kWidth / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ u32x4 load16(const bf16* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// Weights are streamed once per step: a non-temporal hint keeps them from
// evicting the small activation vectors every block re-reads.
__device__ __forceinline__ u32x4 load16_stream(const bf16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Device-coherent access.  Data one block writes and another block of the same
// launch reads (activations, attention partials, the KV cache, the step
// counters) goes through these.  Device-scope loads miss the per-CU L1 and the
// per-XCD L2 for those lines and device-scope stores write through, so crossing
// a grid barrier needs no L2 writeback/invalidate -- only each wave's wait for
// its own stores (stores_done).  Bases must be wave-uniform (a kernel argument).
// ---------------------------------------------------------------------------
constexpr int kCoherent = 16;  // buffer cache-policy bits: device scope (sc1)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, -1, 0x00020000);
}
__device__ __forceinline__ u32x4 coh_ld16(const void* base, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rsrc(base), byte_off, 0, kCoherent);
}
__device__ __forceinline__ void coh_st16(void* base, uint32_t byte_off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rsrc(base), byte_off, 0, kCoherent);
}
__device__ __forceinline__ bf16 coh_ld_bf16(const bf16* base, uint32_t idx) {
  return __builtin_amdgcn_raw_buffer_load_b16(rsrc(base), idx * 2u, 0, kCoherent);
}
__device__ __forceinline__ void coh_st_bf16(bf16* base, uint32_t idx, bf16 v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, rsrc(base), idx * 2u, 0, kCoherent);
}
__device__ __forceinline__ float coh_ldf(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_stf(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int coh_ldi(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_sti(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_sti64(int64_t* p, int64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// This wave's memory operations have completed (stores are visible device-wide).
__device__ __forceinline__ void stores_done() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ float dot8(const u32x4 w, const u32x4 x, float acc) {
  acc = fmaf(bf_lo(w.x), bf_lo(x.x), acc);
  acc = fmaf(bf_hi(w.x), bf_hi(x.x), acc);
  acc = fmaf(bf_lo(w.y), bf_lo(x.y), acc);
  acc = fmaf(bf_hi(w.y), bf_hi(x.y), acc);
  acc = fmaf(bf_lo(w.z), bf_lo(x.z), acc);
  acc = fmaf(bf_hi(w.z), bf_hi(x.z), acc);
  acc = fmaf(bf_lo(w.w), bf_lo(x.w), acc);
  acc = fmaf(bf_hi(w.w), bf_hi(x.w), acc);
  return acc;
}

// ---------------------------------------------------------------------------
// Activation vector in registers.  A wave's lane `l` owns 16-byte chunks
// l, l+64, l+128, ... of a length-K bf16 vector (K % 8 == 0); kCmax bounds the
// chunks per lane (K <= kCmax * 512).
// ---------------------------------------------------------------------------
// Loads are unconditional from clamped in-bounds addresses and masked
// afterwards: a load under a divergent branch makes the wait-count pass fall
// back to waiting for every outstanding load at the join.
template <int kCmax>
__device__ __forceinline__ void load_x(const bf16* __restrict__ x, int nch, int lane,
                                       u32x4 (&xr)[kCmax]) {
#pragma unroll
  for (int i = 0; i < kCmax; ++i) {
    const int c = i * kWave + lane;
    const u32x4 v = load16(x + (int64_t)(c < nch ? c : nch - 1) * 8);
    xr[i] = c < nch ? v : u32x4{0u, 0u, 0u, 0u};
  }
}

// The same, for an activation another block produced (device-coherent loads).
template <int kCmax>
__device__ __forceinline__ void load_x_coh(const bf16* __restrict__ x, int nch, int lane,
                                           u32x4 (&xr)[kCmax]) {
#pragma unroll
  for (int i = 0; i < kCmax; ++i) {
    const int c = i * kWave + lane;
    const u32x4 v = coh_ld16(x, (uint32_t)(c < nch ? c : nch - 1) * 16u);
    xr[i] = c < nch ? v : u32x4{0u, 0u, 0u, 0u};
  }
}

// The Qwen3 RMSNorm (model.py:134-137): xn = bf16(bf16(x * rsqrt(mean(x^2)+eps)) * gamma),
// computed by one wave over the whole vector.  Split in two so a caller can
// issue the x / gamma loads, then its weight loads, and only then wait for x:
// memory counters retire in order, so x must be requested first.
template <int kCmax>
__device__ __forceinline__ void rms_norm_apply(u32x4 (&xr)[kCmax], const u32x4 (&gr)[kCmax], int K,
                                               float eps) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kCmax; ++i) {
    const uint32_t w[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = bf_lo(w[e]), b = bf_hi(w[e]);
      ss += a * a;
      ss += b * b;
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
  for (int i = 0; i < kCmax; ++i) {
    const uint32_t w[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
    const uint32_t gw[4] = {gr[i].x, gr[i].y, gr[i].z, gr[i].w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = rbf(rbf(bf_lo(w[e]) * r) * bf_lo(gw[e]));
      const float hi = rbf(rbf(bf_hi(w[e]) * r) * bf_hi(gw[e]));
      o[e] = pack2(lo, hi);
    }
    xr[i] = u32x4{o[0], o[1], o[2], o[3]};   // chunks past K stay zero (0 * r * 0)
  }
}

template <int kCmax>
__device__ __forceinline__ void rms_norm_x(const bf16* __restrict__ x,
                                           const bf16* __restrict__ gamma, int K, float eps,
                                           int lane, u32x4 (&xr)[kCmax]) {
  const int nch = K / 8;
  u32x4 gr[kCmax];
  load_x<kCmax>(x, nch, lane, xr);
  load_x<kCmax>(gamma, nch, lane, gr);
  rms_norm_apply<kCmax>(xr, gr, K, eps);
}

// Issue the loads of kR consecutive rows of W (row-major [N][K] bf16): lane l
// gets chunks l, l+64, ... of each row.  Weights do not depend on the
// activation, so callers issue these before anything that waits on memory.
template <int kCmax, int kR>
__device__ __forceinline__ void load_rows(const bf16* __restrict__ W, int K, int nch, int64_t row0,
                                          int nvalid, int lane, u32x4 (&w)[kR][kCmax]) {
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    // rows past the end re-read the last valid row; their sums are never stored
    const bf16* rowp = W + (row0 + (r < nvalid ? r : nvalid - 1)) * (int64_t)K;
#pragma unroll
    for (int i = 0; i < kCmax; ++i) {
      const int c = i * kWave + lane;
      // chunks past K re-read a valid chunk; x is zero there, so they add 0
      w[r][i] = load16_stream(rowp + (int64_t)(c < nch ? c : nch - 1) * 8);
    }
  }
  // keep every weight load ahead of the arithmetic that follows: the scheduler
  // otherwise interleaves them with it and fewer bytes are in flight
  __builtin_amdgcn_sched_barrier(0);
}

// Row dot products of loaded weights with the wave's x chunks (all lanes get
// every row's sum).
template <int kCmax, int kR>
__device__ __forceinline__ void dot_loaded(const u32x4 (&w)[kR][kCmax], const u32x4 (&xr)[kCmax],
                                           float (&acc)[kR]) {
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < kCmax; ++i) a = dot8(w[r][i], xr[i], a);
    acc[r] = wave_sum(a);
  }
}

template <int kCmax, int kR>
__device__ __forceinline__ void dot_rows(const bf16* __restrict__ W, int K, int nch, int64_t row0,
                                         int nvalid, const u32x4 (&xr)[kCmax], int lane,
                                         float (&acc)[kR]) {
  u32x4 w[kR][kCmax];
  load_rows<kCmax, kR>(W, K, nch, row0, nvalid, lane, w);
  dot_loaded<kCmax, kR>(w, xr, acc);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// Error flags a kernel raises instead of touching memory it was not given.
enum DeviceError : int {
  kErrNone = 0,
  kErrTokenRange = 1,      // a token id outside [0, vocab)
  kErrPosRange = 2,        // a position past the rope table or the page table
  kErrPageRange = 4,       // a page-table entry outside the pool
  kErrStepRange = 8,       // a step past the sample buffer
  kErrBarrier = 16,        // a grid barrier waited past its bound
};

__device__ __forceinline__ void raise_error(int* err, int code) {
  if (err) atomicOr(err, code);
}

}  // namespace tfd
