// Batched decode step (up to 32 sequences per step), bf16, for gfx950.
//
// The same HIR semantics as the batch-1 kernels (every matmul an f32 sum
// rounded once to bf16, the attention chain rounded where the HIR rounds), laid
// out for a batch: activations are [rows][n] row-major with explicit leading
// dimensions, every sequence has its own position and page-table row, and the
// projections are skinny GEMMs on the matrix cores (16x16x32 bf16 MFMA): at 32
// rows a projection is a real contraction (2 flops per weight byte per row), so
// the VALU dot path would be compute-bound before HBM is.
//
// Kernels of one layer (workload C3: Qwen3-1.7B at batch 32):
//   rmsnorm_rows                 x -> bf16 normalised rows
//   gemm_skinny<STORE>           xn @ [q|k|v]^T            -> qkv   [B][HQ*D+2*HKV*D]
//   attn_rope_scores_batched     per (split, kv head, sequence), as the batch-1 phase
//   attn_pv_combine_batched      per (split, kv head, sequence), last block merges
//   gemm_skinny<RESID>           attn @ Wo^T + residual    -> h1
//   rmsnorm_rows, gemm_skinny<SWIGLU>, gemm_skinny<RESID> (down)
// and per step: rmsnorm_rows (final), gemm_skinny<LOGITS> (bf16-valued f32
// logits), argmax_rows, finalize_rows (pick, next token, position, embedding).

#include <mutex>
#include <type_traits>

#include "decode_phases.h"
#include "host_common.h"
#include "tf_decode.h"

using namespace tfd;
using namespace tfd_host;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxRows = 32;      // one skinny GEMM covers two 16-row MFMA tiles

// Activations that feed a skinny GEMM (the normalised rows, the attention
// output, the SwiGLU output) are stored in the matrix cores' A-operand order,
// 32 rows x K: for 32-wide k step s and 16-row half h, a 1 KiB block at
// (2 s + h) KiB whose 16 bytes at l * 16 hold X[16 h + l % 16][32 s + 8 (l / 16)
// .. +7].  A wave then loads one step's operand as one contiguous KiB.  Rows
// past the batch are never written; they only feed output rows that are not
// stored.
__device__ __forceinline__ int64_t xp_off(int m, int k) {
  return ((int64_t)((k >> 5) * 2 + (m >> 4)) * 64 + (m & 15) + 16 * ((k >> 3) & 3)) * 8 +
         (k & 7);
}

// ---------------------------------------------------------------------------
// Row-wise RMSNorm (model.py:125-137 on each sequence's hidden state): one
// wave per row, the batch-1 arithmetic.  kSingle: the HIR's rms_norm op
// (ir/hir/nn/rms_norm.py:103-110, one rounding after gamma).
// ---------------------------------------------------------------------------
template <int kCmax, bool kSingle = false>
__global__ __launch_bounds__(kWave) void k_rmsnorm_rows(const bf16* __restrict__ x, int ldx,
                                                        const bf16* __restrict__ gamma,
                                                        bf16* __restrict__ out_rows, int ldo,
                                                        bf16* __restrict__ out_packed, int n,
                                                        float eps) {
  const int lane = threadIdx.x;
  const int m = blockIdx.x;
  const bf16* xr_p = x + (int64_t)m * ldx;
  u32x4 xr[kCmax];
  rms_norm_x<kCmax, kSingle>(xr_p, gamma, n, eps, lane, xr);
  const int nch = n / 8;
#pragma unroll
  for (int i = 0; i < kCmax; ++i) {
    const int c = i * kWave + lane;
    if (c < nch) {
      if (out_rows)
        *reinterpret_cast<u32x4*>(out_rows + (int64_t)m * ldo + (int64_t)c * 8) = xr[i];
      if (out_packed) *reinterpret_cast<u32x4*>(out_packed + xp_off(m, c * 8)) = xr[i];
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny GEMM: Y[m][n] = sum_k X[m][k] W[n][k] for m < M <= 32, W packed in
// MFMA order (k_pack_skinny).
//
// At 32 rows the weights are the only large operand (X is at most 32 x 6144
// bf16), so the kernel keeps X stationary: a block stages its K slice of X
// ([rows][Ks], rows = 16 or 32) in LDS once, and its eight waves then stream
// 16-row tiles of W past it -- every weight byte is read once from HBM and X is
// read from L2 once per block, not once per tile.  A wave owns whole tiles (all
// Ks of them), so no cross-wave reduction is needed; with kDepth 32-wide k
// steps (1 KiB per wave each) of weights in flight it crosses tile boundaries
// without draining.  Blocks are persistent over a contiguous range of tiles.
//
// MFMA operand layout of v_mfma_f32_16x16x32_bf16: lane l holds
// A[l % 16][8 (l / 16) .. +7], B[8 (l / 16) .. +7][l % 16] and gets
// D[4 (l / 16) .. +3][l % 16]; A is X (rows) from LDS, B is W^T (16 bytes of one
// weight row per lane).
//
// K is split into `slices` (grid.y) when there are too few tiles to fill the
// chip (o and down: 128 tiles).  Each slice's wave stores its f32 tile in
// fragment order (1 KiB per 16-row half, coalesced), bumps the tile's counter,
// and the wave that arrives last adds the slices in slice order -- so the sum
// does not depend on which slice finishes first -- applies the epilogue and
// puts the counter back to zero for the next call.
// ---------------------------------------------------------------------------
// kSkResidScaled: out = bf16(resid + bf16(y * rmul)), a scaled residual add;
// kSkLogitsDiv: out (f32) = bf16(y / rmul), logits over a published divisor
enum SkinnyEpi {
  kSkStore = 0, kSkResid = 1, kSkSwiglu = 2, kSkLogits = 3, kSkResidF32 = 4, kSkResidScaled = 5,
  kSkLogitsDiv = 6
};

// Two shapes: Ks <= 1024 (66 KiB of LDS, two blocks of four waves per compute
// unit, eight steps in flight per wave) and Ks <= 2048 (the head: one block of
// eight waves per compute unit, sixteen steps in flight per wave when Ks is a
// multiple of 512).


template <int kEpi>
__device__ __forceinline__ void skinny_store(const f32x4 (&c)[2], int halves, int tile, int lane,
                                             int M, int N, const bf16* __restrict__ resid,
                                             int ldr, void* __restrict__ out, int ldo,
                                             float rmul = 1.f) {
  const int r = lane & 15, kq = lane >> 4;
  const int n = tile * 16 + r;
  for (int h = 0; h < halves; ++h) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 16 * h + 4 * kq + e;
      const float y = rbf(c[h][e]);
      if (kEpi == kSkSwiglu) {
        // (gate, up) pairs sit in adjacent columns: lanes r and r ^ 1; the
        // product feeds the down projection, so it is stored in operand order
        const float u = __shfl_xor(y, 1, kWave);
        if ((r & 1) == 0 && m < M && n + 1 < N)
          ((bf16*)out)[xp_off(m, n / 2)] = f2bf(rbf(silu_f(y)) * u);
      } else if (m < M && n < N) {
        if (kEpi == kSkStore)
          ((bf16*)out)[(int64_t)m * ldo + n] = f2bf(y);
        else if (kEpi == kSkResid)
          ((bf16*)out)[(int64_t)m * ldo + n] = f2bf(bf2f(resid[(int64_t)m * ldr + n]) + y);
        else if (kEpi == kSkResidF32)   // f32 residual stream: out = resid + y (in place allowed)
          ((float*)out)[(int64_t)m * ldo + n] =
              reinterpret_cast<const float*>(resid)[(int64_t)m * ldr + n] + y;
        else if (kEpi == kSkResidScaled)   // (in place allowed)
          ((bf16*)out)[(int64_t)m * ldo + n] =
              f2bf(bf2f(resid[(int64_t)m * ldr + n]) + rbf(y * rmul));
        else if (kEpi == kSkLogitsDiv)
          ((float*)out)[(int64_t)m * ldo + n] = rbf(y / rmul);
        else
          ((float*)out)[(int64_t)m * ldo + n] = y;
      }
    }
  }
}

// Weights in MFMA order: for 16-row tile t and 32-wide k step s, a 1 KiB block
// at (t * K/32 + s) KiB whose 16 bytes at l * 16 are
// W[16 t + l % 16][32 s + 8 (l / 16) .. +7] -- the B operand of lane l -- so
// the GEMM's weight loads are whole contiguous KiBs.  Rows past N are zero.
__global__ __launch_bounds__(kBlock) void k_pack_skinny(const bf16* __restrict__ W, int ldw,
                                                        int N, int K, bf16* __restrict__ out,
                                                        int64_t chunks) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= chunks) return;
  const int l = (int)(i & 63);
  const int64_t blk = i >> 6;
  const int ks = K / 32;
  const int64_t t = blk / ks;
  const int st = (int)(blk % ks);
  const int64_t row = t * 16 + (l & 15);
  const u32x4 v = row < N ? load16(W + row * ldw + st * 32 + 8 * (l >> 4)) : u32x4{0u, 0u, 0u, 0u};
  *reinterpret_cast<u32x4*>(out + i * 8) = v;
}

template <int kEpi, int kKsMax, int kWaves, int kDepth>
__global__ __launch_bounds__(kWaves * kWave) void k_gemm_skinny(
    const bf16* __restrict__ X, const bf16* __restrict__ W, int M, int K, int N, int Ks,
    const bf16* __restrict__ resid, int ldr, void* __restrict__ out, int ldo,
    float* __restrict__ part, int* __restrict__ counters, float rmul) {
  constexpr int kThreads = kWaves * kWave;
  __shared__ __align__(16) bf16 xs[32 * kKsMax];
  const int lane = threadIdx.x & (kWave - 1);
  // wave-uniform (scalar) so the tile and step loops branch on scalars
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane & 15, kq = lane >> 4;
  const int halves = M > 16 ? 2 : 1;
  const int slices = gridDim.y, slice = blockIdx.y;
  const int kbase = slice * Ks;
  const int ntiles = (N + 15) / 16;
  const int t0 = (int)((int64_t)blockIdx.x * ntiles / gridDim.x);
  const int t1 = (int)((int64_t)(blockIdx.x + 1) * ntiles / gridDim.x);
  const int steps = Ks / 32;                 // a multiple of kDepth
  const int first = t0 + wave;
  const int ntw = first < t1 ? (t1 - first + kWaves - 1) / kWaves : 0;

  // Load cursor over this wave's (tile, step) sequence in the packed weights:
  // one step of one tile is 1 KiB, lane l's 16 bytes at l * 16 (a wave's load is
  // contiguous).  A wave without tiles reads its block's first tile.
  int lt = first < t1 ? first : (t0 < ntiles ? t0 : ntiles - 1), lk = 0;
  const int ksteps = K / 32;
  const bf16* wbase = W + (int64_t)(kbase / 32) * 512 + lane * 8;
  auto load_next = [&]() {
    const u32x4 v = load16_stream(wbase + ((int64_t)lt * ksteps + lk) * 512);
    const bool wrap = lk + 1 == steps;
    lk = wrap ? 0 : lk + 1;
    lt = wrap ? lt + kWaves : lt;
    return v;
  };
  u32x4 b[kDepth];
#pragma unroll
  for (int u = 0; u < kDepth; ++u) b[u] = load_next();   // in flight while X is staged
  // the X slice (operand-order blocks of steps kbase/32 ..) -> LDS, a plain copy
  {
    const bf16* xsrc = X + (int64_t)(kbase / 32) * 1024;
    const int nchunks = Ks * 4;                // 16-byte chunks: 32 rows x Ks / 8
    constexpr int kB = 8;
    for (int c0 = threadIdx.x; c0 < nchunks; c0 += kB * kThreads) {
      u32x4 v[kB];
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int c = c0 + j * kThreads;
        v[j] = load16(xsrc + (int64_t)(c < nchunks ? c : 0) * 8);
      }
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int c = c0 + j * kThreads;
        if (c < nchunks) *reinterpret_cast<u32x4*>(&xs[c * 8]) = v[j];
      }
    }
  }
  __syncthreads();

  const bf16* xa = xs + lane * 8;
  f32x4 c[2];
  // kDepth steps from LDS x the weights in flight; with kRefill each slot is
  // reloaded with the step kDepth ahead right behind its use (the wave's last
  // chunk has nothing ahead, so it loads nothing)
  auto chunk = [&](int k0, auto refill) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      const bf16* xk = xa + (k0 + u) * 1024;
      const bf16x8_t bw = __builtin_bit_cast(bf16x8_t, b[u]);
      c[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8_t*>(xk), bw,
                                                     c[0], 0, 0, 0);
      c[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          *reinterpret_cast<const bf16x8_t*>(xk + 512), bw, c[1], 0, 0, 0);
      if (decltype(refill)::value) b[u] = load_next();
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int t = 0; t < ntw; ++t) {
    const int tile = first + t * kWaves;
    c[0] = f32x4{0.f, 0.f, 0.f, 0.f};
    c[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int kend = (t + 1 == ntw) ? steps - kDepth : steps;
    for (int k0 = 0; k0 < kend; k0 += kDepth) chunk(k0, std::true_type{});
    if (t + 1 == ntw) chunk(steps - kDepth, std::false_type{});
    bool mine = true;
    if (slices > 1) {
      // this slice's tile in fragment order: [slice][tile][half][lane] x 16 bytes
      const uint32_t own = ((uint32_t)(slice * ntiles + tile) * 2u) * 1024u + lane * 16u;
      for (int h = 0; h < halves; ++h)
        coh_st16(part, own + h * 1024u, __builtin_bit_cast(u32x4, c[h]));
      stores_done();
      int ticket = 0;
      if (lane == 0) ticket = atomicAdd(&counters[tile], 1);
      ticket = __shfl(ticket, 0, kWave);
      mine = ticket == slices - 1;
      if (mine) {
        // the last arrival adds the slices in slice order (four at a time in
        // flight) and re-arms the counter
        f32x4 sum[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        for (int s0 = 0; s0 < slices; s0 += 4) {
          u32x4 v[4][2];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int sl = s0 + j < slices ? s0 + j : slices - 1;
            const uint32_t off = ((uint32_t)(sl * ntiles + tile) * 2u) * 1024u + lane * 16u;
            v[j][0] = coh_ld16(part, off);
            v[j][1] = coh_ld16(part, off + 1024u);   // written only when halves == 2
          }
          // every load is consumed (a select, not a branch), so none is left
          // in flight into registers the next tile reuses
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool valid = s0 + j < slices;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const f32x4 x = __builtin_bit_cast(f32x4, v[j][h]);
#pragma unroll
              for (int e = 0; e < 4; ++e) sum[h][e] += valid ? x[e] : 0.f;
            }
          }
        }
        c[0] = sum[0];
        c[1] = sum[1];
        if (lane == 0) coh_sti(&counters[tile], 0);
      }
    }
    if (mine) skinny_store<kEpi>(c, halves, tile, lane, M, N, resid, ldr, out, ldo, rmul);
  }
}

// ---------------------------------------------------------------------------
// Skinny GEMM for few tiles (the q/k/v, o, gate/up and down projections at
// N / 16 <= a few per compute unit): one block per kT consecutive 16-column
// tiles, its kKW waves splitting K evenly.  Wave w streams the packed weights
// of its K range for its tiles and reads the matching operand-order X blocks
// straight into registers (no other wave needs them, so nothing is staged),
// kDepth steps in flight; the waves' sums meet in LDS and are added in wave
// order.  No partial ever leaves the block, so the launch is one round trip
// of loads plus a barrier -- what the narrow projections need, whose weights
// alone do not keep the chip busy for long.
// ---------------------------------------------------------------------------
// fp8-e4m3fn weights: the same block order at one byte per value (512-byte
// blocks, lane l's 8 bytes at l * 8); gfx950 decodes e4m3fn exactly, every
// value is exact in bf16, so the products and the f32 sums are those of the
// bf16 path, and the output channel's scale multiplies the sum.
template <bool kFp8>
struct SkW {
  using Raw = u32x4;
  static __device__ __forceinline__ Raw load(const void* base, int64_t block, int lane) {
    return load16_stream((const bf16*)base + block * 512 + lane * 8);
  }
  static __device__ __forceinline__ bf16x8_t value(const Raw& r) {
    return __builtin_bit_cast(bf16x8_t, r);
  }
};
template <>
struct SkW<true> {
  using Raw = u32x2;
  static __device__ __forceinline__ Raw load(const void* base, int64_t block, int lane) {
    return __builtin_nontemporal_load(
        reinterpret_cast<const u32x2*>((const uint8_t*)base + block * 512 + lane * 8));
  }
  // gfx950's scaled fp8 -> bf16 pair conversion with scale 1.0 decodes every
  // e4m3fn code exactly (checked over all 256 codes); `sel` picks bytes 2-3
  static __device__ __forceinline__ bf16x8_t value(const Raw& r) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    const bf16x2_v v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.x, 1.0f, false);
    const bf16x2_v v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.x, 1.0f, true);
    const bf16x2_v v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.y, 1.0f, false);
    const bf16x2_v v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.y, 1.0f, true);
    const bf16x8_t o = {v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
    return o;
  }
};

__global__ __launch_bounds__(kBlock) void k_pack_skinny_fp8(const uint8_t* __restrict__ W, int ldw,
                                                            int N, int K,
                                                            uint8_t* __restrict__ out,
                                                            int64_t chunks) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= chunks) return;
  const int l = (int)(i & 63);
  const int64_t blk = i >> 6;
  const int ks = K / 32;
  const int64_t t = blk / ks;
  const int st = (int)(blk % ks);
  const int64_t row = t * 16 + (l & 15);
  u32x2 v = {0u, 0u};
  if (row < N) v = *reinterpret_cast<const u32x2*>(W + row * ldw + st * 32 + 8 * (l >> 4));
  *reinterpret_cast<u32x2*>(out + i * 8) = v;
}

template <int kEpi, int kT, int kKW, int kDepth, bool kFp8 = false, int kH = 2>
__global__ __launch_bounds__(kKW * kWave) void k_gemm_ksplit(
    const bf16* __restrict__ X, const void* __restrict__ W, int M, int K, int N,
    const bf16* __restrict__ resid, int ldr, void* __restrict__ out, int ldo,
    const float* __restrict__ wscale, float* __restrict__ part, int* __restrict__ counters,
    float rmul) {
  using WL = SkW<kFp8>;
  __shared__ f32x4 red[kKW][kT][2][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int ntiles = (N + 15) / 16;
  const int tile0 = blockIdx.x * kT;
  const int slices = gridDim.y, slice = blockIdx.y;   // K slices across blocks
  const int ksteps = K / 32;
  const int steps = ksteps / slices / kKW;   // per wave, a multiple of kDepth
  const int s0 = slice * (ksteps / slices) + wave * steps;
  // X in operand order: step k's two 16-row halves are consecutive KiBs.  A
  // lane whose row is past M reads row M - 1's chunk instead (its outputs are
  // never stored), so a few-row batch loads only its own rows' bytes.
  const int xr0 = min(lane & 15, M - 1), xr1 = min(16 + (lane & 15), M - 1) - 16;
  const bf16* xa = X + (int64_t)s0 * 1024 + (xr0 + 16 * (lane >> 4)) * 8;
  const bf16* xb1 = X + (int64_t)s0 * 1024 + 512 + ((xr1 < 0 ? 0 : xr1) + 16 * (lane >> 4)) * 8;
  int64_t wt[kT];                            // block index of (tile, step s0)
#pragma unroll
  for (int t = 0; t < kT; ++t) {
    const int tt = tile0 + t < ntiles ? tile0 + t : ntiles - 1;
    wt[t] = (int64_t)tt * ksteps + s0;
  }
  typename WL::Raw b[kDepth][kT];
  u32x4 a0[kDepth], a1[kDepth];
  auto issue = [&](int u, int k) {
#pragma unroll
    for (int t = 0; t < kT; ++t) b[u][t] = WL::load(W, wt[t] + k, lane);
    a0[u] = load16(xa + (int64_t)k * 1024);
    if (kH == 2) a1[u] = load16(xb1 + (int64_t)k * 1024);        // rows 16..31
  };
#pragma unroll
  for (int u = 0; u < kDepth; ++u) {
    issue(u, u);
    __builtin_amdgcn_sched_barrier(0);        // issue in step order
  }
  f32x4 c[kT][2];
#pragma unroll
  for (int t = 0; t < kT; ++t) c[t][0] = c[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  // each slot is refilled with the step kDepth ahead right behind its use; the
  // last chunk has nothing ahead (a separate copy, so no branch sits between a
  // load and its use)
  auto chunk = [&](int k0, auto refill) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      const bf16x8_t x0 = __builtin_bit_cast(bf16x8_t, a0[u]);
      const bf16x8_t x1 = __builtin_bit_cast(bf16x8_t, kH == 2 ? a1[u] : a0[u]);
#pragma unroll
      for (int t = 0; t < kT; ++t) {
        const bf16x8_t bw = WL::value(b[u][t]);
        c[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x0, bw, c[t][0], 0, 0, 0);
        if (kH == 2) c[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, bw, c[t][1], 0, 0, 0);
      }
      if (decltype(refill)::value) issue(u, k0 + kDepth + u);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int k0 = 0; k0 + kDepth < steps; k0 += kDepth) chunk(k0, std::true_type{});
  chunk(steps - kDepth, std::false_type{});
#pragma unroll
  for (int t = 0; t < kT; ++t) {
    red[wave][t][0][lane] = c[t][0];
    red[wave][t][1][lane] = c[t][1];
  }
  __syncthreads();
  if (wave >= kT) return;
  // wave t adds the K ranges of tile t in wave order and applies the epilogue
  const int t = wave;
  if (tile0 + t >= ntiles) return;
  f32x4 sum[2] = {red[0][t][0][lane], red[0][t][1][lane]};
#pragma unroll
  for (int w = 1; w < kKW; ++w) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 v = red[w][t][h][lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[h][e] += v[e];
    }
  }
  if (slices > 1) {
    // this slice's tile in fragment order ([slice][tile][half][lane] x 16
    // bytes); the last block to arrive adds the slices in slice order
    const int tile = tile0 + t;
    const uint32_t own = ((uint32_t)(slice * ntiles + tile) * 2u) * 1024u + lane * 16u;
#pragma unroll
    for (int h = 0; h < kH; ++h) coh_st16(part, own + h * 1024u, __builtin_bit_cast(u32x4, sum[h]));
    stores_done();
    int ticket = 0;
    if (lane == 0) ticket = atomicAdd(&counters[tile], 1);
    ticket = __shfl(ticket, 0, kWave);
    if (ticket != slices - 1) return;
#pragma unroll
    for (int h = 0; h < 2; ++h) sum[h] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int sl = 0; sl < slices; ++sl) {
      const uint32_t off = ((uint32_t)(sl * ntiles + tile) * 2u) * 1024u + lane * 16u;
#pragma unroll
      for (int h = 0; h < kH; ++h) {
        const f32x4 x = __builtin_bit_cast(f32x4, coh_ld16(part, off + h * 1024u));
#pragma unroll
        for (int e = 0; e < 4; ++e) sum[h][e] += x[e];
      }
    }
    if (lane == 0) coh_sti(&counters[tile], 0);
  }
  if (kFp8) {
    // every lane holds one output column: its channel's scale
    const int n = (tile0 + t) * 16 + (lane & 15);
    const float sc = wscale[n < N ? n : N - 1];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[h][e] *= sc;
  }
  skinny_store<kEpi>(sum, M > 16 ? 2 : 1, tile0 + t, lane, M, N, resid, ldr, out, ldo, rmul);
}

// ---------------------------------------------------------------------------
// Attention for a batch: grid (nsplit, kv heads, sequences); sequence b has its
// own position, page-table row, QKV row and workspaces.  The phase bodies are
// the batch-1 ones.
// ---------------------------------------------------------------------------
// Tiles per split: `chunks` when positive; when 0, derived from the sequence's
// position so that its prior context spreads evenly over the nsplit splits
// (both launches of a step read the same position, so they agree on it).
__device__ __forceinline__ int split_chunks(int chunks, int P, int max_pages, int nsplit) {
  if (chunks > 0) return chunks;
  const int Pc = (P >= 0 && P < max_pages * kPage) ? P : 0;
  const int tiles = (Pc + kSplit - 1) / kSplit;
  const int c = (tiles + nsplit - 1) / nsplit;
  return c > 0 ? c : 1;
}

template <int D, int G>
__global__ __launch_bounds__(kBlock) void k_attn_scores_b(
    const bf16* __restrict__ qkv, int ldq, const bf16* __restrict__ gq,
    const bf16* __restrict__ gk, const bf16* __restrict__ cos_t, const bf16* __restrict__ sin_t,
    int rope_rows, const int* __restrict__ pos, const int* __restrict__ page_table, int max_pages,
    bf16* __restrict__ kpool, bf16* __restrict__ vpool, int num_pages, int kv_heads, float scale,
    float eps, float* __restrict__ S, int s_stride, float* __restrict__ smax,
    float* __restrict__ snew, int chunks, int* err) {
  const int b = blockIdx.z, heads = kv_heads * G, nsplit = gridDim.x;
  const int P = coh_ldi(pos + b);
  const int* pt = page_table + (int64_t)b * max_pages;
  chunks = split_chunks(chunks, P, max_pages, nsplit);
  KTile<D> kt;
  k_tile_issue_at<D, false>(blockIdx.x * chunks * kSplit, blockIdx.y, P, pt, max_pages, kpool,
                     num_pages, kv_heads, kt);
  const QKPre pre = qk_prefetch<D, G>(P, P, gq, gk, cos_t, sin_t, rope_rows, pt, max_pages);
  __shared__ __attribute__((aligned(16))) uint32_t hs[(G + 2) * D / 2];
  stage_head<D, G>(blockIdx.y, heads, kv_heads, qkv + (int64_t)b * ldq, hs);
  __syncthreads();
  attn_scores_phase<D, G, false>(blockIdx.x, blockIdx.y, hs, pre, rope_rows, P, P, pt,
                                 max_pages, kpool, vpool, num_pages, kv_heads, scale, eps,
                                 S + (int64_t)b * heads * s_stride, s_stride,
                                 smax + (int64_t)b * nsplit * heads, snew + (int64_t)b * heads,
                                 AttnLL{}, kt, err, chunks);
}

// Attention output of sequence b in operand order (it feeds the o projection).
struct PackedOut {
  int b;
  __device__ uint32_t operator()(int k) const { return (uint32_t)xp_off(b, k); }
};

template <int D, int G>
__global__ __launch_bounds__(kBlock) void k_attn_pv_b(
    const bf16* __restrict__ qkv, int ldq, const int* __restrict__ pos,
    const int* __restrict__ page_table, int max_pages, const bf16* __restrict__ vpool,
    int num_pages, int kv_heads, const float* __restrict__ S, int s_stride,
    const float* __restrict__ smax, const float* __restrict__ snew, float* part_sum,
    float* part_out, int* counters, bf16* __restrict__ attn_out, int chunks, int* err) {
  const int b = blockIdx.z, heads = kv_heads * G, nsplit = gridDim.x;
  int P = coh_ldi(pos + b);
  if (P < 0 || P >= max_pages * kPage) P = 0;
  const int* pt = page_table + (int64_t)b * max_pages;
  chunks = split_chunks(chunks, P, max_pages, nsplit);
  VTile<D> vt;
  v_tile_issue_at<D, false>(blockIdx.x * chunks * kSplit, blockIdx.y, P, pt, max_pages, vpool,
                     num_pages, kv_heads, vt);
  attn_pv_phase<D, G, false, NoHook, PackedOut>(
      blockIdx.x, blockIdx.y, nsplit, qkv + (int64_t)b * ldq, P, pt, max_pages, vpool,
      num_pages, kv_heads, S + (int64_t)b * heads * s_stride, s_stride,
      smax + (int64_t)b * nsplit * heads, snew + (int64_t)b * heads,
      part_sum + (int64_t)b * nsplit * heads, part_out + (int64_t)b * nsplit * heads * D,
      counters + (int64_t)b * kv_heads, attn_out, AttnLL{}, vt, err, chunks, NoHook{},
      PackedOut{b});
}

// ---------------------------------------------------------------------------
// Greedy pick per row (generation.py:24-26: the first maximal bf16 logit) and
// the step's last node per sequence (the batch form of finalize_phase).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_argmax_rows(const float* __restrict__ logits, int ldl,
                                                      int V, int* __restrict__ pick) {
  const float* row = logits + (int64_t)blockIdx.x * ldl;
  float b = kNegInf;
  int i = 0x7fffffff;
  for (int k = threadIdx.x; k < V; k += blockDim.x) {
    const float v = row[k];
    if (better(v, k, b, i)) {
      b = v;
      i = k;
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
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = b;
    si[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bb = sv[0];
    int ii = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      if (better(sv[w], si[w], bb, ii)) {
        bb = sv[w];
        ii = si[w];
      }
    pick[blockIdx.x] = (ii >= 0 && ii < V) ? ii : 0;   // an all-NaN row has no pick
  }
}

// The same pick in two stages for long rows: kArgChunks blocks per row each
// find their chunk's first maximum, then one wave per row picks the first
// maximum among the chunk winners (ties go to the lower index: the chunks are
// in index order and `better` prefers the lower index).
constexpr int kArgChunks = 64;

__global__ __launch_bounds__(kBlock) void k_argmax_chunks(const float* __restrict__ logits,
                                                          int ldl, int V,
                                                          int* __restrict__ part) {
  const int row = blockIdx.y, chunk = blockIdx.x;
  const int per = (V + kArgChunks - 1) / kArgChunks;
  const int k0 = chunk * per;
  const int k1 = (k0 + per < V) ? k0 + per : V;
  const float* r = logits + (int64_t)row * ldl;
  float b = kNegInf;
  int i = 0x7fffffff;
  for (int k = k0 + (int)threadIdx.x; k < k1; k += kBlock) {
    const float v = r[k];
    if (better(v, k, b, i)) {
      b = v;
      i = k;
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
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = b;
    si[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWavesPerBlock; ++w)
      if (better(sv[w], si[w], b, i)) {
        b = sv[w];
        i = si[w];
      }
    part[((int64_t)row * kArgChunks + chunk) * 2] = __float_as_int(b);
    part[((int64_t)row * kArgChunks + chunk) * 2 + 1] = i;
  }
}

__global__ __launch_bounds__(kWave) void k_argmax_pick(const int* __restrict__ part, int V,
                                                       int* __restrict__ pick) {
  const int row = blockIdx.x, lane = threadIdx.x;
  float b = __int_as_float(part[((int64_t)row * kArgChunks + lane) * 2]);
  int i = part[((int64_t)row * kArgChunks + lane) * 2 + 1];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ob = __shfl_xor(b, m, kWave);
    const int oi = __shfl_xor(i, m, kWave);
    if (better(ob, oi, b, i)) {
      b = ob;
      i = oi;
    }
  }
  if (lane == 0) pick[row] = (i >= 0 && i < V) ? i : 0;   // an all-NaN row has no pick
}

__global__ __launch_bounds__(kBlock) void k_finalize_rows(
    const int* __restrict__ pick, const int* __restrict__ inp, int ld_inp,
    const int* __restrict__ plen, int64_t* __restrict__ ids, int* __restrict__ pos,
    int* __restrict__ sam, int ld_sam, int nsteps, const bf16* __restrict__ table,
    bf16* __restrict__ hid, int ldh, int hidden, int vocab, int* err) {
  const int b = blockIdx.x;
  __shared__ int next_s;
  if (threadIdx.x == 0) {
    const int p = pos[b];
    const int ii = pick[b];
    int next = ii;
    if (p < 0 || p >= nsteps) {
      raise_error(err, kErrStepRange);
    } else {
      sam[(int64_t)b * ld_sam + p] = ii;
      if (p + 1 < plen[b] && p + 1 < nsteps) next = inp[(int64_t)b * ld_inp + p + 1];
    }
    if (next < 0 || next >= vocab) {
      raise_error(err, kErrTokenRange);
      next = 0;
    }
    ids[b] = next;
    pos[b] = p + 1;
    next_s = next;
  }
  __syncthreads();
  const bf16* row = table + (int64_t)next_s * hidden;
  bf16* o = hid + (int64_t)b * ldh;
  for (int c = threadIdx.x; c < hidden / 8; c += kBlock)
    *reinterpret_cast<u32x4*>(o + (int64_t)c * 8) = load16(row + (int64_t)c * 8);
}

__global__ __launch_bounds__(kBlock) void k_embed_rows(const bf16* __restrict__ table,
                                                       const int64_t* __restrict__ ids,
                                                       bf16* __restrict__ out, int ldo,
                                                       int hidden, int vocab, int* err) {
  int64_t id = ids[blockIdx.x];
  if (id < 0 || id >= vocab) {
    if (threadIdx.x == 0) raise_error(err, kErrTokenRange);
    id = 0;
  }
  const bf16* row = table + id * (int64_t)hidden;
  bf16* o = out + (int64_t)blockIdx.x * ldo;
  for (int c = threadIdx.x; c < hidden / 8; c += kBlock)
    *reinterpret_cast<u32x4*>(o + (int64_t)c * 8) = load16(row + (int64_t)c * 8);
}

}  // namespace

#define TFD_ATTN_SWITCH_B(D, G, CALL)                                      \
  if (D == 128 && G == 2) { constexpr int kD = 128, kG = 2; CALL; }        \
  else if (D == 64 && G == 2) { constexpr int kD = 64, kG = 2; CALL; }     \
  else if (D == 128 && G == 1) { constexpr int kD = 128, kG = 1; CALL; }   \
  else return fail(kUnsupported, "attention: head_dim=%d group=%d not built", D, G);

extern "C" {

int tfd_rmsnorm_rows_bf16(const void* x, int ldx, const void* gamma, void* out, int ldo,
                          int rows, int n, float eps, int packed, void* stream) {
  if (!x || !gamma || !out) return fail(kBadArg, "rmsnorm_rows: null pointer");
  if (rows <= 0 || n <= 0 || n % 8 || ldx < n || ldx % 8 ||
      (packed ? (rows > kMaxRows || n % 32) : (ldo < n || ldo % 8)))
    return fail(kBadShape, "rmsnorm_rows: rows=%d n=%d ldx=%d ldo=%d packed=%d", rows, n, ldx,
                ldo, packed);
  auto s = (hipStream_t)stream;
  bf16* o_rows = packed ? nullptr : (bf16*)out;
  bf16* o_packed = packed ? (bf16*)out : nullptr;
  TFD_CMAX_SWITCH(n, hipLaunchKernelGGL((k_rmsnorm_rows<kC>), dim3(rows), dim3(kWave), 0, s,
                                        (const bf16*)x, ldx, (const bf16*)gamma, o_rows, ldo,
                                        o_packed, n, eps));
  return launched("rmsnorm_rows");
}

int tfd_rmsnorm_rows2_bf16(const void* x, int ldx, const void* gamma, void* out_rows, int ldo,
                           void* out_packed, int rows, int n, float eps, void* stream) {
  if (!x || !gamma || (!out_rows && !out_packed))
    return fail(kBadArg, "rmsnorm_rows2: null pointer");
  if (rows <= 0 || n <= 0 || n % 8 || ldx < n || ldx % 8 ||
      (out_packed && (rows > kMaxRows || n % 32)) || (out_rows && (ldo < n || ldo % 8)))
    return fail(kBadShape, "rmsnorm_rows2: rows=%d n=%d ldx=%d ldo=%d", rows, n, ldx, ldo);
  auto s = (hipStream_t)stream;
  TFD_CMAX_SWITCH(n, hipLaunchKernelGGL((k_rmsnorm_rows<kC>), dim3(rows), dim3(kWave), 0, s,
                                        (const bf16*)x, ldx, (const bf16*)gamma, (bf16*)out_rows,
                                        ldo, (bf16*)out_packed, n, eps));
  return launched("rmsnorm_rows2");
}

int tfd_tf_rmsnorm_rows_bf16(const void* x, int ldx, const void* gamma, void* out_rows, int ldo,
                             void* out_packed, int rows, int n, float eps, void* stream) {
  if (!x || !gamma || (!out_rows && !out_packed))
    return fail(kBadArg, "tf_rmsnorm_rows: null pointer");
  if (rows <= 0 || n <= 0 || n % 8 || ldx < n || ldx % 8 ||
      (out_packed && (rows > kMaxRows || n % 32)) || (out_rows && (ldo < n || ldo % 8)))
    return fail(kBadShape, "tf_rmsnorm_rows: rows=%d n=%d ldx=%d ldo=%d", rows, n, ldx, ldo);
  auto s = (hipStream_t)stream;
  TFD_CMAX_SWITCH(n, hipLaunchKernelGGL((k_rmsnorm_rows<kC, true>), dim3(rows), dim3(kWave), 0,
                                        s, (const bf16*)x, ldx, (const bf16*)gamma,
                                        (bf16*)out_rows, ldo, (bf16*)out_packed, n, eps));
  return launched("tf_rmsnorm_rows");
}

}  // extern "C"

namespace {

// Launch shape of one skinny GEMM.  K is split into a power-of-two number of
// slices until there are at least four tile-slices per compute unit (each slice
// a multiple of 256 deep and at most 2048, the LDS stage); blocks are
// persistent over tiles, one or two per compute unit.
struct SkinnyPlan {
  int slices, Ks, blocks_per_slice;
  bool wide;                // Ks > 1024: the 2048-deep LDS stage
  int64_t work_floats;      // counters + partials
};


// The work buffer starts with kSkCounters tile counters (zero before first use;
// every call leaves the ones it used at zero) at a fixed place, so GEMMs of
// different shapes can share one buffer; the f32 partials follow.
constexpr int kSkCounters = TFD_SKINNY_COUNTERS;

int64_t skinny_work(int ntiles, int slices) {
  return slices == 1 ? 0 : (int64_t)kSkCounters + (int64_t)slices * ntiles * 512;
}

SkinnyPlan skinny_plan(int K, int N, int64_t work_floats) {
  const int ntiles = (N + 15) / 16;
  const int cus = compute_units();
  int s = 1;
  while (K / s > 2048 && K % (512 * s) == 0) s *= 2;
  while ((int64_t)ntiles * s < 4 * cus && K % (512 * s) == 0) s *= 2;
  while (s > 1 && (skinny_work(ntiles, s) > work_floats || ntiles > kSkCounters)) s /= 2;
  SkinnyPlan p;
  p.slices = s;
  p.Ks = K / s;
  p.wide = p.Ks > 1024;
  const int per_cu = p.wide ? 1 : 2;
  const int waves = p.wide ? 8 : 4;
  int64_t bps = ((int64_t)ntiles + waves - 1) / waves;
  const int64_t cap = ((int64_t)per_cu * cus + s - 1) / s;
  if (bps > cap) bps = cap;
  p.blocks_per_slice = (int)(bps < 1 ? 1 : bps);
  p.work_floats = skinny_work(ntiles, s);
  return p;
}

// Which kernel: tiles per block of the K-split kernel, or 0 for the
// X-stationary one.  The K-split kernel takes the projections with few tiles
// (it needs no partials outside the block) and any K deeper than the LDS stage;
// the X-stationary kernel takes the head, whose many tiles fill the chip and
// whose X is worth keeping in LDS across them.  A block takes two tiles of a
// wide shape when the batch is at most 16 rows (one X half per step), one
// otherwise (measured: M = 32 gate/up 1% faster per step with one, M = 1 and 16
// about 1% slower).
int ksplit_tiles(int M, int K, int N) {
  const int ntiles = (N + 15) / 16;
  if (K > 2048 || ntiles < 4 * compute_units()) return ntiles >= 512 && M <= 16 ? 2 : 1;
  return 0;
}

}  // namespace

extern "C" {

int tfd_pack_skinny_bf16(const void* w, int ldw, int N, int K, void* packed, void* stream) {
  if (!w || !packed) return fail(kBadArg, "pack_skinny: null pointer");
  if (N <= 0 || K <= 0 || K % 256 || ldw < K || ldw % 8)
    return fail(kBadShape, "pack_skinny: N=%d K=%d (multiple of 256) ldw=%d", N, K, ldw);
  const int64_t chunks = (int64_t)(N + 15) / 16 * (K / 32) * 64;
  hipLaunchKernelGGL(k_pack_skinny, dim3((unsigned)((chunks + kBlock - 1) / kBlock)),
                     dim3(kBlock), 0, (hipStream_t)stream, (const bf16*)w, ldw, N, K,
                     (bf16*)packed, chunks);
  return launched("pack_skinny");
}

int tfd_pack_skinny_fp8(const void* w, int ldw, int N, int K, void* packed, void* stream) {
  if (!w || !packed) return fail(kBadArg, "pack_skinny_fp8: null pointer");
  if (N <= 0 || K <= 0 || K % 256 || ldw < K || ldw % 8)
    return fail(kBadShape, "pack_skinny_fp8: N=%d K=%d (multiple of 256) ldw=%d", N, K, ldw);
  const int64_t chunks = (int64_t)(N + 15) / 16 * (K / 32) * 64;
  hipLaunchKernelGGL(k_pack_skinny_fp8, dim3((unsigned)((chunks + kBlock - 1) / kBlock)),
                     dim3(kBlock), 0, (hipStream_t)stream, (const uint8_t*)w, ldw, N, K,
                     (uint8_t*)packed, chunks);
  return launched("pack_skinny_fp8");
}

// the scaled residual epilogue's code inside this file (not a public epilogue:
// its multiplier comes through tfd_gemm_skinny_fp8_resid_scaled)
constexpr int kEpiResidScaled = -1;

static int gemm_skinny_fp8(const void* x, const void* w, const float* scale, int M, int K, int N,
                           int epilogue, const void* resid, int ldr, float rmul, void* out,
                           int ldo, void* stream) {
  if (!x || !w || !scale || !out) return fail(kBadArg, "gemm_skinny_fp8: null pointer");
  if (M <= 0 || M > kMaxRows || K <= 0 || K % 256 || N <= 0)
    return fail(kBadShape, "gemm_skinny_fp8: M=%d (1..32) K=%d (multiple of 256) N=%d", M, K, N);
  if ((epilogue == TFD_EPI_RESID || epilogue == TFD_EPI_RESID_F32 ||
       epilogue == kEpiResidScaled) && (!resid || ldr < N))
    return fail(kBadArg, "gemm_skinny_fp8: residual epilogue needs resid with ldr >= N");
  if (epilogue == TFD_EPI_SWIGLU ? (N % 2 || (N / 2) % 32) : ldo < N)
    return fail(kBadShape, "gemm_skinny_fp8: ldo=%d N=%d", ldo, N);
  auto s = (hipStream_t)stream;
  auto xb = (const bf16*)x;
  auto rb = (const bf16*)resid;
  const int ntiles = (N + 15) / 16;
  const int steps = K / 32 / 8;
  const dim3 grid(ntiles);
#define TFD_KSPLIT8(EPI, D)                                                                   \
  if (M <= 16)                                                                                \
    hipLaunchKernelGGL((k_gemm_ksplit<EPI, 1, 8, D, true, 1>), grid, dim3(8 * kWave), 0, s, xb, \
                       w, M, K, N, rb, ldr, out, ldo, scale, nullptr, nullptr, rmul);               \
  else                                                                                        \
    hipLaunchKernelGGL((k_gemm_ksplit<EPI, 1, 8, D, true, 2>), grid, dim3(8 * kWave), 0, s, xb, \
                       w, M, K, N, rb, ldr, out, ldo, scale, nullptr, nullptr, rmul)
#define TFD_KSPLIT8_EPI(EPI)                    \
  if (steps % 8 == 0) TFD_KSPLIT8(EPI, 8);      \
  else if (steps % 4 == 0) TFD_KSPLIT8(EPI, 4); \
  else if (steps % 2 == 0) TFD_KSPLIT8(EPI, 2); \
  else TFD_KSPLIT8(EPI, 1);
  switch (epilogue) {
    case TFD_EPI_STORE: TFD_KSPLIT8_EPI(kSkStore); break;
    case TFD_EPI_RESID: TFD_KSPLIT8_EPI(kSkResid); break;
    case TFD_EPI_SWIGLU: TFD_KSPLIT8_EPI(kSkSwiglu); break;
    case TFD_EPI_LOGITS: TFD_KSPLIT8_EPI(kSkLogits); break;
    case TFD_EPI_RESID_F32: TFD_KSPLIT8_EPI(kSkResidF32); break;
    case kEpiResidScaled: TFD_KSPLIT8_EPI(kSkResidScaled); break;
    default:
      return fail(kBadArg, "gemm_skinny_fp8: epilogue %d", epilogue);
  }
#undef TFD_KSPLIT8_EPI
#undef TFD_KSPLIT8
  return launched("gemm_skinny_fp8");
}

int tfd_gemm_skinny_fp8(const void* x, const void* w, const float* scale, int M, int K, int N,
                        int epilogue, const void* resid, int ldr, void* out, int ldo,
                        void* stream) {
  if (epilogue == kEpiResidScaled) return fail(kBadArg, "gemm_skinny_fp8: epilogue %d", epilogue);
  return gemm_skinny_fp8(x, w, scale, M, K, N, epilogue, resid, ldr, 1.f, out, ldo, stream);
}

int tfd_gemm_skinny_fp8_resid_scaled(const void* x, const void* w, const float* scale, int M,
                                     int K, int N, const void* resid, int ldr, float mult,
                                     void* out, int ldo, void* stream) {
  return gemm_skinny_fp8(x, w, scale, M, K, N, kEpiResidScaled, resid, ldr, mult, out, ldo,
                         stream);
}

}  // extern "C"

namespace {

constexpr int kEpiLogitsDiv = -2;   // internal: tfd_gemm_skinny_bf16_logits_div

int gemm_skinny_bf16(const void* x, const void* w, int M, int K, int N, int epilogue,
                     const void* resid, int ldr, void* out, int ldo, float* work,
                     int64_t work_floats, float rmul, void* stream) {
  if (!x || !w || !out) return fail(kBadArg, "gemm_skinny: null pointer");
  if (M <= 0 || M > kMaxRows || K <= 0 || K % 256 || N <= 0)
    return fail(kBadShape, "gemm_skinny: M=%d (1..32) K=%d (multiple of 256) N=%d", M, K, N);
  if ((epilogue == TFD_EPI_RESID || epilogue == TFD_EPI_RESID_F32) && (!resid || ldr < N))
    return fail(kBadArg, "gemm_skinny: residual epilogue needs resid with ldr >= N");
  if (epilogue == TFD_EPI_SWIGLU ? (N % 2 || (N / 2) % 32) : ldo < N)
    return fail(kBadShape, "gemm_skinny: ldo=%d N=%d (SwiGLU: N/2 a multiple of 32)", ldo, N);
  if (work_floats < 0 || (work_floats > 0 && !work))
    return fail(kBadArg, "gemm_skinny: work=%p with %lld floats", (void*)work,
                (long long)work_floats);
  auto s = (hipStream_t)stream;
  auto xb = (const bf16*)x;
  auto wb = (const bf16*)w;
  auto rb = (const bf16*)resid;
  const int ntiles = (N + 15) / 16;
  const int kt = ksplit_tiles(M, K, N);
  if (kt > 0) {
    dim3 grid((ntiles + kt - 1) / kt);
    // fewer blocks than compute units: with a work buffer, K is also split
    // across blocks (slices, added by the last block to finish a tile);
    // without one, sixteen waves split K instead of eight
    int slices = 1;
    if (kt == 1 && work) {
      for (int sl = 4; sl >= 2; sl /= 2)
        if ((int)grid.x * sl <= compute_units() && (K / 32) % (sl * 8) == 0 &&
            work_floats >= kSkCounters + (int64_t)sl * ntiles * 512 && ntiles <= kSkCounters) {
          slices = sl;
          break;
        }
    }
    grid.y = slices;
    int* counters = slices > 1 ? (int*)work : nullptr;
    float* part = slices > 1 ? work + kSkCounters : nullptr;
    const int steps = K / 32 / slices / 8;
    const bool wide = slices == 1 && (int)grid.x < compute_units() && (K / 32) % 16 == 0;
    const int steps16 = K / 32 / 16;
#define TFD_KSPLIT(EPI, KT, D)                                                                  \
  if (M <= 16)                                                                                  \
    hipLaunchKernelGGL((k_gemm_ksplit<EPI, KT, 8, D, false, 1>), grid, dim3(8 * kWave), 0, s,   \
                       xb, wb, M, K, N, rb, ldr, out, ldo, nullptr, part, counters, rmul);           \
  else                                                                                          \
    hipLaunchKernelGGL((k_gemm_ksplit<EPI, KT, 8, D, false, 2>), grid, dim3(8 * kWave), 0, s,   \
                       xb, wb, M, K, N, rb, ldr, out, ldo, nullptr, part, counters, rmul)
#define TFD_KSPLIT16(EPI, D)                                                                    \
  if (M <= 16)                                                                                  \
    hipLaunchKernelGGL((k_gemm_ksplit<EPI, 1, 16, D, false, 1>), grid, dim3(16 * kWave), 0, s,  \
                       xb, wb, M, K, N, rb, ldr, out, ldo, nullptr, nullptr, nullptr, rmul);         \
  else                                                                                          \
    hipLaunchKernelGGL((k_gemm_ksplit<EPI, 1, 16, D, false, 2>), grid, dim3(16 * kWave), 0, s,  \
                       xb, wb, M, K, N, rb, ldr, out, ldo, nullptr, nullptr, nullptr, rmul)
#define TFD_KSPLIT_EPI(EPI)                              \
  if (wide && kt == 1 && steps16 % 8 == 0) TFD_KSPLIT16(EPI, 8); \
  else if (wide && kt == 1 && steps16 % 4 == 0) TFD_KSPLIT16(EPI, 4); \
  else if (kt == 2 && steps % 8 == 0) TFD_KSPLIT(EPI, 2, 8);  \
  else if (steps % 8 == 0) TFD_KSPLIT(EPI, 1, 8);        \
  else if (steps % 4 == 0) TFD_KSPLIT(EPI, 1, 4);        \
  else if (steps % 2 == 0) TFD_KSPLIT(EPI, 1, 2);        \
  else TFD_KSPLIT(EPI, 1, 1);
    switch (epilogue) {
      case TFD_EPI_STORE: TFD_KSPLIT_EPI(kSkStore); break;
      case TFD_EPI_RESID: TFD_KSPLIT_EPI(kSkResid); break;
      case TFD_EPI_SWIGLU: TFD_KSPLIT_EPI(kSkSwiglu); break;
      case TFD_EPI_LOGITS: TFD_KSPLIT_EPI(kSkLogits); break;
      case TFD_EPI_RESID_F32: TFD_KSPLIT_EPI(kSkResidF32); break;
      case kEpiLogitsDiv: TFD_KSPLIT_EPI(kSkLogitsDiv); break;
      default:
        return fail(kBadArg, "gemm_skinny: epilogue %d", epilogue);
    }
#undef TFD_KSPLIT_EPI
#undef TFD_KSPLIT16
#undef TFD_KSPLIT
    return launched("gemm_skinny");
  }
  const SkinnyPlan plan = skinny_plan(K, N, work ? work_floats : 0);
  if (plan.Ks > 2048 || plan.Ks % 256)
    return fail(kBadShape, "gemm_skinny: K=%d needs slices of at most 2048 (multiples of 256); "
                "a work buffer of %lld floats allows %d", K, (long long)plan.work_floats,
                plan.slices);
  if ((int64_t)plan.slices * ((N + 15) / 16) * 2048 >= ((int64_t)1 << 31))
    return fail(kBadShape, "gemm_skinny: N=%d with %d K slices", N, plan.slices);
  int* counters = plan.slices > 1 ? (int*)work : nullptr;
  float* part = plan.slices > 1 ? work + kSkCounters : nullptr;
  const dim3 grid(plan.blocks_per_slice, plan.slices);
#define TFD_SKINNY_LAUNCH(EPI)                                                                \
  if (plan.wide && plan.Ks % 512 == 0)                                                        \
    hipLaunchKernelGGL((k_gemm_skinny<EPI, 2048, 8, 16>), grid, dim3(8 * kWave), 0, s, xb,    \
                       wb, M, K, N, plan.Ks, rb, ldr, out, ldo, part, counters, rmul);        \
  else if (plan.wide)                                                                         \
    hipLaunchKernelGGL((k_gemm_skinny<EPI, 2048, 8, 8>), grid, dim3(8 * kWave), 0, s, xb,     \
                       wb, M, K, N, plan.Ks, rb, ldr, out, ldo, part, counters, rmul);        \
  else                                                                                        \
    hipLaunchKernelGGL((k_gemm_skinny<EPI, 1024, 4, 8>), grid, dim3(4 * kWave), 0, s, xb,     \
                       wb, M, K, N, plan.Ks, rb, ldr, out, ldo, part, counters, rmul);
  switch (epilogue) {
    case TFD_EPI_STORE: TFD_SKINNY_LAUNCH(kSkStore); break;
    case TFD_EPI_RESID: TFD_SKINNY_LAUNCH(kSkResid); break;
    case TFD_EPI_SWIGLU: TFD_SKINNY_LAUNCH(kSkSwiglu); break;
    case TFD_EPI_LOGITS: TFD_SKINNY_LAUNCH(kSkLogits); break;
    case TFD_EPI_RESID_F32: TFD_SKINNY_LAUNCH(kSkResidF32); break;
    case kEpiLogitsDiv: TFD_SKINNY_LAUNCH(kSkLogitsDiv); break;
    default:
      return fail(kBadArg, "gemm_skinny: epilogue %d", epilogue);
  }
#undef TFD_SKINNY_LAUNCH
  return launched("gemm_skinny");
}

// The splits reach every cached position and the score rows hold them: fixed
// splits cover nsplit x split_tiles x 64 positions; derived ones (split_tiles
// 0) always cover the prior context, whose scores go at their positions.
bool batched_splits_cover(int max_pages, int nsplit, int split_tiles, int score_stride) {
  const int64_t cap = (int64_t)max_pages * kPage;
  if (split_tiles == 0) return score_stride >= (cap + kSplit - 1) / kSplit * kSplit;
  const int64_t slen = (int64_t)split_tiles * kSplit;
  return nsplit * slen >= cap && score_stride >= nsplit * slen;
}

}  // namespace

extern "C" {

int tfd_gemm_skinny_bf16(const void* x, const void* w, int M, int K, int N, int epilogue,
                         const void* resid, int ldr, void* out, int ldo, float* work,
                         int64_t work_floats, void* stream) {
  if (epilogue == kEpiLogitsDiv) return fail(kBadArg, "gemm_skinny: epilogue %d", epilogue);
  return gemm_skinny_bf16(x, w, M, K, N, epilogue, resid, ldr, out, ldo, work, work_floats, 1.f,
                          stream);
}

int tfd_gemm_skinny_bf16_logits_div(const void* x, const void* w, int M, int K, int N,
                                    float divisor, void* out, int ldo, float* work,
                                    int64_t work_floats, void* stream) {
  if (!(divisor > 0.f)) return fail(kBadArg, "gemm_skinny_logits_div: divisor %g", divisor);
  return gemm_skinny_bf16(x, w, M, K, N, kEpiLogitsDiv, nullptr, 0, out, ldo, work, work_floats,
                          divisor, stream);
}

int tfd_attn_rope_scores_paged_batched(
    const void* qkv, int ldq, const void* gamma_q, const void* gamma_k, const void* cos_table,
    const void* sin_table, int rope_rows, const int32_t* pos, const int32_t* page_table,
    int max_pages, void* k_pool, void* v_pool, int num_pages, int batch, int heads, int kv_heads,
    int head_dim, float scale, float eps, float* scores, int score_stride, float* split_max,
    float* score_new, int nsplit, int split_tiles, int32_t* err, void* stream) {
  if (!qkv || !gamma_q || !gamma_k || !cos_table || !sin_table || !pos || !page_table ||
      !k_pool || !v_pool || !scores || !split_max || !score_new)
    return fail(kBadArg, "attn_rope_scores_batched: null pointer");
  if (batch <= 0 || batch > 65535 || kv_heads <= 0 || heads % kv_heads || nsplit <= 0 ||
      max_pages <= 0 || num_pages <= 0 || split_tiles < 0)
    return fail(kBadShape, "attn_rope_scores_batched: batch=%d heads=%d kv_heads=%d nsplit=%d "
                "split_tiles=%d", batch, heads, kv_heads, nsplit, split_tiles);
  if (!batched_splits_cover(max_pages, nsplit, split_tiles, score_stride) ||
      ldq < (heads + 2 * kv_heads) * head_dim)
    return fail(kBadShape, "attn_rope_scores_batched: nsplit=%d / score_stride=%d / ldq=%d do "
                "not cover the cache", nsplit, score_stride, ldq);
  const int G = heads / kv_heads;
  const dim3 grid(nsplit, kv_heads, batch);
  auto s = (hipStream_t)stream;
  TFD_ATTN_SWITCH_B(head_dim, G,
      hipLaunchKernelGGL((k_attn_scores_b<kD, kG>), grid, dim3(kBlock), 0, s, (const bf16*)qkv,
                         ldq, (const bf16*)gamma_q, (const bf16*)gamma_k,
                         (const bf16*)cos_table, (const bf16*)sin_table, rope_rows, pos,
                         page_table, max_pages, (bf16*)k_pool, (bf16*)v_pool, num_pages,
                         kv_heads, scale, eps, scores, score_stride, split_max, score_new,
                         split_tiles, err));
  return launched("attn_rope_scores_batched");
}

int tfd_attn_pv_combine_paged_batched(
    const void* qkv, int ldq, const int32_t* pos, const int32_t* page_table, int max_pages,
    const void* v_pool, int num_pages, int batch, int heads, int kv_heads, int head_dim,
    const float* scores, int score_stride, const float* split_max, const float* score_new,
    float* part_sum, float* part_out, int nsplit, int split_tiles, int32_t* counters,
    void* attn_out, int32_t* err, void* stream) {
  if (!qkv || !pos || !page_table || !v_pool || !scores || !split_max || !score_new ||
      !part_sum || !part_out || !counters || !attn_out)
    return fail(kBadArg, "attn_pv_combine_batched: null pointer");
  if (batch <= 0 || batch > kMaxRows || kv_heads <= 0 || heads % kv_heads || nsplit <= 0 ||
      max_pages <= 0 || num_pages <= 0 || (heads * head_dim) % 32 || split_tiles < 0)
    return fail(kBadShape, "attn_pv_combine_batched: batch=%d (1..32) heads=%d kv_heads=%d "
                "nsplit=%d split_tiles=%d", batch, heads, kv_heads, nsplit, split_tiles);
  if (!batched_splits_cover(max_pages, nsplit, split_tiles, score_stride))
    return fail(kBadShape, "attn_pv_combine_batched: nsplit=%d does not cover the cache", nsplit);
  const int G = heads / kv_heads;
  const dim3 grid(nsplit, kv_heads, batch);
  auto s = (hipStream_t)stream;
  TFD_ATTN_SWITCH_B(head_dim, G,
      hipLaunchKernelGGL((k_attn_pv_b<kD, kG>), grid, dim3(kBlock), 0, s, (const bf16*)qkv, ldq,
                         pos, page_table, max_pages, (const bf16*)v_pool, num_pages, kv_heads,
                         scores, score_stride, split_max, score_new, part_sum, part_out,
                         counters, (bf16*)attn_out, split_tiles, err));
  return launched("attn_pv_combine_batched");
}

int tfd_argmax_rows(const float* logits, int ldl, int rows, int vocab, int32_t* pick,
                    int32_t* work, void* stream) {
  if (!logits || !pick) return fail(kBadArg, "argmax_rows: null pointer");
  if (rows <= 0 || rows > 65535 || vocab <= 0 || ldl < vocab)
    return fail(kBadShape, "argmax_rows: rows=%d vocab=%d ldl=%d", rows, vocab, ldl);
  auto s = (hipStream_t)stream;
  if (!work) {
    hipLaunchKernelGGL(k_argmax_rows, dim3(rows), dim3(1024), 0, s, logits, ldl, vocab, pick);
  } else {
    hipLaunchKernelGGL(k_argmax_chunks, dim3(kArgChunks, rows), dim3(kBlock), 0, s, logits, ldl,
                       vocab, work);
    hipLaunchKernelGGL(k_argmax_pick, dim3(rows), dim3(kWave), 0, s, work, vocab, pick);
  }
  return launched("argmax_rows");
}

int tfd_finalize_rows(const int32_t* pick, int rows, const int32_t* inp, int ld_inp,
                      const int32_t* prompt_len, int64_t* ids, int32_t* pos, int32_t* sam,
                      int ld_sam, int nsteps, const void* table, void* hid, int ldh, int hidden,
                      int vocab, int32_t* err, void* stream) {
  if (!pick || !inp || !prompt_len || !ids || !pos || !sam || !table || !hid)
    return fail(kBadArg, "finalize_rows: null pointer");
  if (rows <= 0 || nsteps <= 0 || ld_inp < nsteps || ld_sam < nsteps || hidden <= 0 ||
      hidden % 8 || ldh < hidden || ldh % 8 || vocab <= 0)
    return fail(kBadShape, "finalize_rows: rows=%d nsteps=%d hidden=%d ldh=%d", rows, nsteps,
                hidden, ldh);
  hipLaunchKernelGGL(k_finalize_rows, dim3(rows), dim3(kBlock), 0, (hipStream_t)stream, pick,
                     inp, ld_inp, prompt_len, ids, pos, sam, ld_sam, nsteps, (const bf16*)table,
                     (bf16*)hid, ldh, hidden, vocab, err);
  return launched("finalize_rows");
}

int tfd_embed_rows_bf16(const void* table, const int64_t* ids, void* out, int ldo, int rows,
                        int hidden, int vocab, int32_t* err, void* stream) {
  if (!table || !ids || !out) return fail(kBadArg, "embed_rows: null pointer");
  if (rows <= 0 || hidden <= 0 || hidden % 8 || ldo < hidden || ldo % 8 || vocab <= 0)
    return fail(kBadShape, "embed_rows: rows=%d hidden=%d ldo=%d", rows, hidden, ldo);
  hipLaunchKernelGGL(k_embed_rows, dim3(rows), dim3(kBlock), 0, (hipStream_t)stream,
                     (const bf16*)table, ids, (bf16*)out, ldo, hidden, vocab, err);
  return launched("embed_rows");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The skinny GEMM for callers that cannot allocate (code under graph capture,
// serving loops, harnesses that forbid hipMalloc): its K-split work -- tile
// counters and f32 partial tiles -- lives in a file-scope device array instead
// of a caller-supplied buffer.  Each device holds its own copy of the array for
// the life of the process; its address on the current device is looked up once
// (hipGetSymbolAddress: the array's name is not a device address in host code).
// The array is zero when the code object loads (a __device__ array without an
// initializer), and every call leaves the tile counters it used at zero, as
// with a caller's buffer, so nothing is ever enqueued to clear it: a first call
// made under stream capture behaves as any other.  Calls that overlap on one
// device share the array and race.
// ---------------------------------------------------------------------------
namespace {

constexpr int64_t kScratchPartials = (int64_t)1 << 21;            // 8 MiB of f32 tiles
constexpr int64_t kScratchFloats = kSkCounters + kScratchPartials;

__device__ __align__(256) float scratch[kScratchFloats];

constexpr int kScratchDevices = 64;
float* g_scratch[kScratchDevices] = {};
std::mutex g_scratch_lock;

// The current device's scratch, looked up on first use; nullptr (rc set by
// fail()) when that fails.
float* scratch_on_device(int& rc) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    rc = fail((int)e, "gemm_skinny_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kScratchDevices) {
    rc = fail(kUnsupported, "gemm_skinny_noalloc: device %d past the %d this library tracks",
              dev, kScratchDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      rc = fail(e != hipSuccess ? (int)e : kUnsupported,
                "gemm_skinny_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = (float*)p;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" {

int tfd_gemm_skinny_bf16_noalloc(const void* x, const void* w, int M, int K, int N,
                                 int epilogue, const void* resid, int ldr, void* out, int ldo,
                                 void* stream) {
  if (M <= 0 || M > kMaxRows || K <= 0 || K % 256 || N <= 0)
    return fail(kBadShape, "gemm_skinny_noalloc: M=%d (1..32) K=%d (multiple of 256) N=%d", M,
                K, N);
  // No shape needs more than the scratch: K deeper than one LDS stage goes to the
  // K-split kernel, which needs no partials, and a split across blocks is
  // planned within the scratch's size (fewer slices when it would not fit), as
  // the work-buffer entry plans within its caller's buffer.
  if (epilogue == kEpiLogitsDiv) return fail(kBadArg, "gemm_skinny_noalloc: epilogue %d", epilogue);
  int rc = 0;
  float* work = scratch_on_device(rc);
  if (!work) return rc;
  return gemm_skinny_bf16(x, w, M, K, N, epilogue, resid, ldr, out, ldo, work, kScratchFloats,
                          1.f, stream);
}

}  // extern "C"
