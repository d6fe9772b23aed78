// Device-side building blocks shared by every decode kernel (gfx950, wave64).
//
// Numerics contract.  The authored Qwen3 HIR (examples/qwen3_1_7b-tilelang/
// ref_src/model.py:125-234) rounds to bf16 after every op it declares at bf16,
// and the reference evaluator computes each such op in f32 and rounds once
// (torch CPU semantics for bf16 tensors).  The helpers below reproduce that:
//   * rbf(x)   rounds an f32 to the nearest-even bf16 and back (c10::BFloat16's
//              rule for every non-NaN value);
//   * the file is compiled with -ffp-contract=off so `a * b + c` stays two
//     rounded ops, as two torch ops are; fused arithmetic (the packed bf16 dot)
//     is used only in matmul accumulations, whose order is not the reference's
//     anyway;
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

// f32 -> bf16 with round-to-nearest-even: gfx950's packed convert instruction
// (v_cvt_pk_bf16_f32), which rounds as c10::BFloat16 does for every finite value
// and infinity (tests/test_gpu_rounding.py checks it against torch bit for bit).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16 f2bf(float f) { return __builtin_bit_cast(bf16, (__bf16)f); }
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// acc + bf16(p0) + bf16(p1): the two products are rounded to bf16 by one
// conversion and added to the f32 accumulator by one dot instruction against
// (1, 1) -- the HIR's "round each product, sum in f32" at two VALU operations
// per pair instead of six (the sum's association differs, as any f32 order may).
__device__ __forceinline__ float add_rounded2(float acc, float p0, float p1) {
  const bf16x2_t r = {(__bf16)p0, (__bf16)p1};
  const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(r, one, acc, false);
}

// Cross-lane reductions.  Within a row of 16 lanes the partner values come
// from DPP (quad_perm xor 1, xor 2, row_half_mirror, row_mirror: VALU operand
// modifiers, no LDS traffic); across rows from ds_bpermute.  Every step adds a
// value to its partner's, and a + b == b + a, so all participating lanes end
// with the same bits.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within 16

// Across the two 16-lane rows of each 32-lane half, and across the two halves:
// gfx950's lane-swap instructions (v_permlane16_swap / v_permlane32_swap) hand
// every lane both values of its pair in registers, no LDS round trip.  With
// both operands the same vector, result [0] holds the pair's lower member and
// [1] the upper one in every lane.
__device__ __forceinline__ void pair16(float v, float& lo, float& hi) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair32(float v, float& lo, float& hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}

// Sum within aligned groups of `width` lanes (width a power of two <= 64).
template <int kWidth>
__device__ __forceinline__ float group_sum(float v) {
  if (kWidth >= 2) v += dpp_f<kDppXor1>(v);
  if (kWidth >= 4) v += dpp_f<kDppXor2>(v);
  if (kWidth >= 8) v += dpp_f<kDppHalfMirror>(v);
  if (kWidth >= 16) v += dpp_f<kDppMirror>(v);
  if (kWidth >= 32) {
    // v_i + v_(i^16), the pair's two members in either order (the same bits)
    float lo, hi;
    pair16(v, lo, hi);
    v = lo + hi;
  }
  if (kWidth >= 64) {
    float lo, hi;
    pair32(v, lo, hi);
    v = lo + hi;
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<kWave>(v); }

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  float lo, hi;
  pair16(v, lo, hi);
  v = fmaxf(lo, hi);
  pair32(v, lo, hi);
  return fmaxf(lo, hi);
}

// Every pointer these helpers take is device (global) memory.  Saying so keeps
// the compiler from emitting FLAT loads for pointers it read from memory (the
// per-layer weight tables): a FLAT load also counts against the LDS/scalar
// counter, so the next LDS read or scalar load would wait for it.
typedef const __attribute__((address_space(1))) u32x4 g_u32x4;
__device__ __forceinline__ u32x4 load16(const bf16* p) {
  return *(g_u32x4*)(p);
}
// Weights are streamed once per step: a non-temporal hint keeps them from
// evicting the small activation vectors every block re-reads.
__device__ __forceinline__ u32x4 load16_stream(const bf16* p) {
  return __builtin_nontemporal_load((g_u32x4*)(p));
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

// The base is read through readfirstlane: a pointer the kernel loaded from
// memory (the per-layer weight table) sits in vector registers, and a buffer
// descriptor the compiler must treat as divergent costs a loop around every
// access (one pass per distinct descriptor value among the lanes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  void* u = (void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, -1, 0x00020000);
}
// A descriptor of `bytes` bytes: a load at an offset past them returns zeros
// without a memory access (kOutOfRange is such an offset for any buffer under
// 2 GiB, with room to add steps to it).
constexpr uint32_t kOutOfRange = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_bounded(const void* base, uint32_t bytes) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  void* u = (void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, (int)bytes, 0x00020000);
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

// Dot product of two 16-byte chunks (8 bf16 each) accumulated into f32 with
// the packed bf16 dot instruction: two exact bf16 products and the running sum
// per instruction, four instructions per chunk.  Used only where the HIR has an
// f32-accumulated matmul (the summation order there is not the reference's
// anyway); products the HIR rounds to bf16 one by one are written out instead.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}
__device__ __forceinline__ float dot8(const u32x4 w, const u32x4 x, float acc) {
  acc = dot2(w.x, x.x, acc);
  acc = dot2(w.y, x.y, acc);
  acc = dot2(w.z, x.z, acc);
  acc = dot2(w.w, x.w, acc);
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
// kSingle selects the HIR's own rms_norm op instead (src/tilefoundry/ir/hir/nn/
// rms_norm.py:103-110: f32(f32(x * r) * gamma) rounded to bf16 once), the norm
// the Granite model writes as tf.rms_norm.
// The scale 1 / sqrt(mean(x^2) + eps) of a vector held as below (chunks past K
// zero): the sum of squares in lane-chunk order, then the wave sum.
template <int kCmax>
__device__ __forceinline__ float rms_scale(const u32x4 (&xr)[kCmax], int K, float eps) {
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
  return 1.0f / sqrtf(ss / (float)K + eps);
}

// One chunk of the normalised vector, given the scale.
template <bool kSingle = false>
__device__ __forceinline__ u32x4 rms_norm_chunk(const u32x4 x, const u32x4 g, float r) {
  const uint32_t w[4] = {x.x, x.y, x.z, x.w};
  const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = kSingle ? (bf_lo(w[e]) * r) * bf_lo(gw[e])
                             : rbf(rbf(bf_lo(w[e]) * r) * bf_lo(gw[e]));
    const float hi = kSingle ? (bf_hi(w[e]) * r) * bf_hi(gw[e])
                             : rbf(rbf(bf_hi(w[e]) * r) * bf_hi(gw[e]));
    o[e] = pack2(lo, hi);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

template <int kCmax, bool kSingle = false>
__device__ __forceinline__ void rms_norm_apply(u32x4 (&xr)[kCmax], const u32x4 (&gr)[kCmax], int K,
                                               float eps) {
  const float r = rms_scale<kCmax>(xr, K, eps);
#pragma unroll
  for (int i = 0; i < kCmax; ++i)
    xr[i] = rms_norm_chunk<kSingle>(xr[i], gr[i], r);   // chunks past K stay zero (0 * r * 0)
}

// The same norm shared by the kWavesPerBlock waves of a block that all hold
// the whole vector (kCmax == kWavesPerBlock): every wave computes the scale
// (the sum's order needs the whole vector per lane), wave w normalises chunk
// slice w into `buf` (kCmax * 256 words of LDS) and every wave reads it back --
// the values rms_norm_apply gives, with a quarter of its per-element work per
// wave.  Every wave of the block must call it (it holds a block barrier).
template <int kCmax>
__device__ __forceinline__ void rms_norm_apply_block(u32x4 (&xr)[kCmax], const u32x4 (&gr)[kCmax],
                                                     int K, float eps, uint32_t* buf) {
  static_assert(kCmax == kWavesPerBlock, "one chunk slice per wave");
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const float r = rms_scale<kCmax>(xr, K, eps);
#pragma unroll
  for (int i = 0; i < kCmax; ++i)
    if (i == wave)
      *reinterpret_cast<u32x4*>(buf + 4 * (i * kWave + lane)) = rms_norm_chunk(xr[i], gr[i], r);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kCmax; ++i) xr[i] = *reinterpret_cast<const u32x4*>(buf + 4 * (i * kWave + lane));
}

template <int kCmax, bool kSingle = false>
__device__ __forceinline__ void rms_norm_x(const bf16* __restrict__ x,
                                           const bf16* __restrict__ gamma, int K, float eps,
                                           int lane, u32x4 (&xr)[kCmax]) {
  const int nch = K / 8;
  u32x4 gr[kCmax];
  load_x<kCmax>(x, nch, lane, xr);
  load_x<kCmax>(gamma, nch, lane, gr);
  rms_norm_apply<kCmax, kSingle>(xr, gr, K, eps);
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

// ---------------------------------------------------------------------------
// The thread group a phase runs on: its thread index (0 .. kBlock-1) and its
// barrier.  Every caller today runs phases on the whole kBlock-thread block.
// ---------------------------------------------------------------------------
struct BlockGrp {
  static __device__ __forceinline__ int tid() { return (int)threadIdx.x; }
  static __device__ __forceinline__ void sync() { __syncthreads(); }
};

// Error flags a kernel raises instead of touching memory it was not given.
enum DeviceError : int {
  kErrNone = 0,
  kErrTokenRange = 1,      // a token id outside [0, vocab)
  kErrPosRange = 2,        // a position past the rope table or the page table
  kErrPageRange = 4,       // a page-table entry outside the pool
  kErrStepRange = 8,       // a step past the sample buffer
  kErrSync = 16,           // a wait for another block's data passed its bound
};

__device__ __forceinline__ void raise_error(int* err, int code) {
  if (err) atomicOr(err, code);
}

// ---------------------------------------------------------------------------
// Flag-in-data words for the persistent kernel.  A word is 8 bytes: a 32-bit
// payload and the 32-bit tag of the (step, layer) that wrote it, written by one
// 8-byte device-coherent store (two words by one 16-byte store, each 8-byte half
// carrying its own tag), so a reader sees the old word or the new one, never a
// mix.  A reader polls until the tag it expects is there: the data is its own
// ready signal, so no barrier, counter or store-completion wait sits between a
// producer and its consumers.  Tags grow over a run and a buffer is rewritten
// only after every reader of its previous contents is done (each rewrite
// depends, through the step's data flow, on outputs that every reader produced
// after reading), so equality is the test.  A wait is bounded: past the bound
// it raises kErrSync, and once the flag is up every other wait gives up too.
// ---------------------------------------------------------------------------
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
constexpr uint32_t kPollBound = 1u << 21;

// Cache policy of an exchange whose writer and readers all run on one XCD.
// Loads are device scope, as kCoherent: the workgroup-scope bit alone does not
// make a load miss the compute unit's L1 when a workgroup stays on one compute
// unit, so a poll through it can keep reading a stale line (measured: such
// polls never completed).  Stores are plain: the L1 writes through to the
// XCD's L2, where a device-scope load of the same XCD finds the line, so the
// word never has to travel to memory and back (measured ping-pong between two
// blocks of one XCD: 0.47 us per round trip, 0.77 us with device-scope stores;
// a block of another XCD never sees such a store, so only intra-XCD exchanges
// use it).  The bit above the cache-policy field marks the policy; ld_bits /
// st_bits give the bits a load / store of the exchange carries.
constexpr int kXcdLocal = kCoherent | (1 << 16);
constexpr int ld_bits(int pol) { return pol & 0xffff; }
constexpr int st_bits(int pol) { return (pol >> 16) != 0 ? 0 : (pol & 0xffff); }

template <int kPol = kCoherent>
__device__ __forceinline__ void ll_put(uint32_t* base, uint32_t word, uint32_t payload,
                                       uint32_t tag) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2{payload, tag}, rsrc(base), word * 8u, 0,
                                        st_bits(kPol));
}
// words `word` and `word + 1` (word even) in one store
template <int kPol = kCoherent>
__device__ __forceinline__ void ll_put2(uint32_t* base, uint32_t word, uint32_t p0, uint32_t p1,
                                        uint32_t tag) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{p0, tag, p1, tag}, rsrc(base), word * 8u, 0,
                                         st_bits(kPol));
}

__device__ __forceinline__ bool ll_give_up(uint32_t& spins, int* err) {
  if ((++spins & 255u) != 0) return false;
  if (spins > kPollBound) {
    raise_error(err, kErrSync);
    return true;
  }
  return (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSync) != 0;
}

// The payloads of words `word`, `word + 1` (word even) once both carry `tag`.
template <int kPol = kCoherent>
__device__ __forceinline__ u32x2 ll_get2(const uint32_t* base, uint32_t word, uint32_t tag,
                                         int* err) {
  u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc(base), word * 8u, 0, ld_bits(kPol));
  uint32_t spins = 0;
  while (v.y != tag || v.w != tag) {
    if (ll_give_up(spins, err)) break;
    // the compiler must issue the load again: without a clobber it may reuse the first result
    __asm__ volatile("" ::: "memory");
    v = __builtin_amdgcn_raw_buffer_load_b128(rsrc(base), word * 8u, 0, ld_bits(kPol));
  }
  return u32x2{v.x, v.z};
}

template <int kPol = kCoherent>
__device__ __forceinline__ uint32_t ll_get(const uint32_t* base, uint32_t word, uint32_t tag,
                                           int* err) {
  u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rsrc(base), word * 8u, 0, ld_bits(kPol));
  uint32_t spins = 0;
  while (v.y != tag) {
    if (ll_give_up(spins, err)) break;
    __asm__ volatile("" ::: "memory");
    v = __builtin_amdgcn_raw_buffer_load_b64(rsrc(base), word * 8u, 0, ld_bits(kPol));
  }
  return v.x;
}

// Stage a flag-in-data bf16 vector of n values (n % 4 == 0) into LDS as plain
// bf16 pairs; the caller synchronises the block before reading it.  Each
// thread issues all its loads of a batch, and while any of them is stale
// issues them all again and checks them all: a batch costs one round trip per
// poll, never one per load.
template <int kPol = kCoherent, class Grp = BlockGrp>
__device__ __forceinline__ void ll_stage(const uint32_t* ll, int n, uint32_t tag,
                                         uint32_t* __restrict__ lds, int* err) {
  constexpr int kBatch = 8;
  const int npairs = n / 4;
  for (int i0 = Grp::tid(); i0 < npairs; i0 += kBlock * kBatch) {
    // loads of this batch the wave needs at all (its first lane has the most),
    // as a wave-uniform count; lanes past the end re-read their first word
    const int first = __builtin_amdgcn_readfirstlane(i0);
    const int kn = (npairs - first + kBlock - 1) / kBlock;
    u32x4 v[kBatch];
    uint32_t spins = 0;
    for (;;) {
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int i = i0 + k * kBlock;
        if (k < kn)
          v[k] = __builtin_amdgcn_raw_buffer_load_b128(
              rsrc(ll), (uint32_t)(i < npairs ? i : i0) * 16u, 0, ld_bits(kPol));
      }
      bool ok = true;
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (k < kn) ok = ok && v[k].y == tag && v[k].w == tag;
      if (ok || ll_give_up(spins, err)) break;
      __asm__ volatile("" ::: "memory");
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int i = i0 + k * kBlock;
      if (i < npairs) {
        lds[2 * i] = v[k].x;
        lds[2 * i + 1] = v[k].z;
      }
    }
  }
}

}  // namespace tfd
