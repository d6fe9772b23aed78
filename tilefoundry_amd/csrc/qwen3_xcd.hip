// The batch-1 Qwen3 decode step partitioned over the 8 XCDs of an MI355X.
//
// The chip is 8 XCDs of 32 compute units.  A 2048-value vector handed from
// every block to all 256 blocks costs ~1.5 us (measured: device-scope polls,
// every load in flight); handed among the 32 blocks of one XCD it costs ~1 us
// (fewer readers of the same lines).  The step is a chain of hand-offs, so
// the kernel keeps most of them inside an XCD: each layer is split across XCDs
// the way tensor parallelism splits it across GPUs, with the XCD as the unit.
//
// A block plays XCD x = its hardware XCC id and rank r = b / 8 among that XCD's
// 32 blocks.  The dispatcher places workgroups round-robin over the XCDs, but
// the XCD it starts a launch on moves from launch to launch (measured: b % 8 is
// not the XCC id after some launches), so x comes from the hardware; under any
// rotation the blocks of one XCD are b = c, c + 8, ..., so b / 8 is a rank.
// Were placement ever not round-robin, some (x, r) would go unplayed, the
// blocks waiting for its outputs would pass their poll bound, and the launch
// would end with kErrSync: a wrong placement cannot produce results that look
// valid.  Per layer, XCD x owns kv head x and its query
// heads 2x, 2x + 1 (the Qwen3-1.7B shape: 16 q heads, 8 kv heads, head_dim 128,
// hidden 2048, intermediate 6144):
//   qkv     the XCD's 512 q/k/v rows (16 per block, full rows of 2048)
//   attn    kv head x over the context in at most 32 contiguous splits of ct
//           64-position tiles, ct = ceil(tiles / 32): split r is rank r's, so
//           a rank's share grows by one tile only when every rank's does.
//           Scores, the split maxima, P.V partials and the merge all exchange
//           inside the XCD (model.py:172-212, the two-pass softmax as authored)
//   o       K split: the XCD's 256 attention outputs against W_o[:, 256x..+256];
//           block r makes rows 64r..64r+63 of that partial product
//   gate/up the XCD's 768 intermediate columns (48 gate/up rows per block)
//   down    K split: the XCD's 768 SwiGLU values against W_down[:, 768x..+768]
// and the o and down products are summed over XCDs by an all-reduce: block
// (x, r) reads the 8 XCDs' partials of rows 64r..64r+63 (device scope), adds
// them in XCD order, applies the residual (h1 = hidden + o, out = h1 + mlp, the
// bf16 roundings of model.py:236-266), and publishes its 64 values to its XCD;
// every block of the XCD then reads the whole vector from the L2.  Every XCD
// sums the same partials in the same order, so all hold the same bits.
//
// Hand-offs per layer: 2 across XCDs (the all-reduces), 6 inside one.  The
// weights of each phase are issued before the wait for its input, as in the
// chip-wide persistent kernel (qwen3_decode.hip); the lm_head and the greedy
// pick are that kernel's.
//
// Replaces the same steps as tfd_decode_persistent (examples/qwen3_1_7b-
// tilelang/fast/engine.py:189-217: one captured step per token).

#include "decode_phases.h"
#include "host_common.h"
#include "tf_decode.h"

#include <stdlib.h>

using namespace tfd;
using namespace tfd_host;

namespace {

constexpr int kXcds = 8;
constexpr int kRanks = 32;                 // blocks per XCD
constexpr int kErrPlacement = 32;          // an XCC id outside 0..7: not the 8-XCD device

// Exchange buffers are arrays of 8-byte (payload, tag) words held as uint32_t:
// word n starts at uint32 2n.
__device__ __forceinline__ uint32_t* word_at(uint32_t* base, int64_t n) { return base + 2 * n; }

__device__ __forceinline__ int xcc_id() {
  int x;
  __asm__ volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x & 0xf;
}

// ---------------------------------------------------------------------------
// K-split slabs (o, down): a wave owns 16 output rows of its block's 64; lane l
// works on row 2p + l / 32 of pass p, with the row's 16-byte chunks c, c + 32,
// ... where c = l % 32 (the slab is kC chunks of 8 per lane and row: 256
// values for o, 768 for down).  Row sums are 32-lane sums.
// ---------------------------------------------------------------------------
template <int kC>
__device__ __forceinline__ void slab_issue(const bf16* __restrict__ W, int ld, int row0, int col0,
                                           u32x4 (&w)[8][kC]) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int half = lane >> 5, c = lane & 31;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int64_t row = row0 + 16 * wave + 2 * p + half;
#pragma unroll
    for (int j = 0; j < kC; ++j) w[p][j] = load16_stream(W + row * ld + col0 + 8 * (c + 32 * j));
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Partial row sums of the slab with x (kC chunks of 8 per lane from LDS, bf16
// pairs) -> f32 words of part (device scope; rows row0 .. row0 + 63).
template <int kC>
__device__ __forceinline__ void slab_finish(const uint32_t* xs, const u32x4 (&w)[8][kC],
                                            uint32_t* part, int row0, uint32_t tag) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int half = lane >> 5, c = lane & 31;
  u32x4 xr[kC];
#pragma unroll
  for (int j = 0; j < kC; ++j) xr[j] = *reinterpret_cast<const u32x4*>(xs + 4 * (c + 32 * j));
  float a[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    a[p] = 0.f;
#pragma unroll
    for (int j = 0; j < kC; ++j) a[p] = dot8(w[p][j], xr[j], a[p]);
  }
  // the eight passes' sums over each 32-lane half at once (rows_sum's
  // exchanges without the first): lane l ends with pass (l / 4) % 8 of its half
  float b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[j]),
                                                    __float_as_uint(a[j + 4]), false, false);
    b[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  const bool b3 = lane & 8, b2 = lane & 4;
  float d[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float keep = b3 ? b[k + 2] : b[k], give = b3 ? b[k] : b[k + 2];
    d[k] = keep + dpp_f<kDppMirror>(give);
  }
  float mine = (b2 ? d[1] : d[0]) + dpp_f<kDppHalfMirror>(b2 ? d[0] : d[1]);
  mine += dpp_f<kDppXor2>(mine);
  mine += dpp_f<kDppXor1>(mine);
  // the first lane of each group of four holds row 2p + half: one word each
  if ((lane & 3) == 0) {
    const int p = (lane >> 2) & 7;
    ll_put<kCoherent>(part, (uint32_t)(row0 + 16 * wave + 2 * p + half), __float_as_uint(mine),
                      tag);
  }
}

// Rows first .. first + kN - 1 of a wave's kRtot gate/up rows (gemv_issue's
// row mapping), so a caller can request some of them early.
template <int kCmax, int kRtot, int kN>
__device__ __forceinline__ void rows_issue(int vb, const bf16* __restrict__ W, int K, int first,
                                           u32x4 (&w)[kN][kCmax]) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row0 = ((int64_t)vb * kWavesPerBlock + wave) * kRtot + first;
  load_rows<kCmax, kN>(W, K, K / 8, row0, kN, lane, w);
}

// The all-reduce of rows r*64 .. r*64+63 of an H-long f32 product held as one
// partial per XCD (part: [8][H] words): sum in XCD order, then out = bf16(res +
// bf16(sum)) for those rows, published to this XCD's copy (bf16 pairs), and
// the whole vector read back into `full` (LDS, H/2 words).  `res` is the
// residual in LDS (bf16 pairs).
__device__ __forceinline__ void allreduce_residual(const uint32_t* part, int H, int r,
                                                   const uint32_t* res, uint32_t* mine_xcd,
                                                   uint32_t* full, uint32_t tag, float* red,
                                                   int* err) {
  const int tid = threadIdx.x;
  {
    const int y = tid / 32, i2 = tid % 32;          // 256 threads: 8 XCDs x 32 word pairs
    const u32x2 v = ll_get2<kCoherent>(part, (uint32_t)(y * H + 64 * r + 2 * i2), tag, err);
    red[y * 64 + 2 * i2] = __uint_as_float(v.x);
    red[y * 64 + 2 * i2 + 1] = __uint_as_float(v.y);
  }
  __syncthreads();
  if (tid < 32) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int y = 0; y < kXcds; ++y) {
      s0 += red[y * 64 + 2 * tid];
      s1 += red[y * 64 + 2 * tid + 1];
    }
    const int w = 32 * r + tid;                      // word of rows 64r + 2 tid, +1
    const uint32_t rw = res[w];
    const uint32_t pr = bf_pair(f2bf(bf_lo(rw) + rbf(s0)), f2bf(bf_hi(rw) + rbf(s1)));
    ll_put<kXcdLocal>(mine_xcd, (uint32_t)w, pr, tag);
  }
  ll_stage<kXcdLocal>(mine_xcd, H, tag, full, err);
  __syncthreads();
}

// The all-reduce's sum for rows kRows q .. kRows q + kRows - 1 of an H-long
// f32 product held as one partial per XCD (part: [8][H] words): sum in XCD
// order, out = bf16(res + bf16(sum)), published to this XCD's copy (bf16
// pairs).  Readers stage the whole vector from there.  The same arithmetic as
// allreduce_residual.
template <int kRows>
__device__ __forceinline__ void allreduce_publish(const uint32_t* part, int H, int q,
                                                  const uint32_t* res, uint32_t* mine_xcd,
                                                  uint32_t tag, float* red, int* err) {
  constexpr int kPairs = kRows / 2;                 // word pairs per XCD partial
  static_assert(kXcds * kPairs % kBlock == 0 && kPairs <= kBlock, "whole passes");
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < kXcds * kPairs / kBlock; ++k) {
    const int i = tid + k * kBlock, y = i / kPairs, i2 = i % kPairs;
    const u32x2 v = ll_get2<kCoherent>(part, (uint32_t)(y * H + kRows * q + 2 * i2), tag, err);
    red[y * kRows + 2 * i2] = __uint_as_float(v.x);
    red[y * kRows + 2 * i2 + 1] = __uint_as_float(v.y);
  }
  __syncthreads();
  if (tid < kPairs) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int y = 0; y < kXcds; ++y) {
      s0 += red[y * kRows + 2 * tid];
      s1 += red[y * kRows + 2 * tid + 1];
    }
    const int w = kPairs * q + tid;                  // word of rows kRows q + 2 tid, +1
    const uint32_t rw = res[w];
    const uint32_t pr = bf_pair(f2bf(bf_lo(rw) + rbf(s0)), f2bf(bf_hi(rw) + rbf(s1)));
    ll_put<kXcdLocal>(mine_xcd, (uint32_t)w, pr, tag);
  }
}

// A slab (slab_issue's lanes and rows) requested straight into LDS: load (p, j)
// of wave w lands as 1 KB at block ((w * 8 + p) * kC + j), lane l's 16 bytes at
// l.  Only for a block that waits on no other block until the data is used:
// a barrier after these loads waits for every load issued before it.
template <int kC>
__device__ __forceinline__ void slab_to_lds(const bf16* __restrict__ W, int ld, int row0, int col0,
                                            u32x4* lds) {
  typedef __attribute__((address_space(1))) void g_void;
  typedef __attribute__((address_space(3))) void l_void;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int half = lane >> 5, c = lane & 31;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int64_t row = row0 + 16 * wave + 2 * p + half;
#pragma unroll
    for (int j = 0; j < kC; ++j)
      __builtin_amdgcn_global_load_lds((g_void*)(W + row * ld + col0 + 8 * (c + 32 * j)),
                                       (l_void*)(lds + ((wave * 8 + p) * kC + j) * kWave), 16, 0,
                                       2 /* nt: streamed once */);
  }
}
template <int kC>
__device__ __forceinline__ void slab_from_lds(const u32x4* lds, u32x4 (&w)[8][kC]) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
#pragma unroll
  for (int p = 0; p < 8; ++p)
#pragma unroll
    for (int j = 0; j < kC; ++j) w[p][j] = lds[((wave * 8 + p) * kC + j) * kWave + lane];
}

__device__ __forceinline__ void stamp(uint64_t*& tl) {
  if (tl && threadIdx.x == 0) *tl++ = wall_clock64();
}

template <int kCmax, int kR>
__device__ __forceinline__ void lm_head_rows(int64_t row0, int V, int lane,
                                             const u32x4 (&xr)[kCmax],
                                             const u32x4 (&w)[kR][kCmax], float* logits,
                                             float& best, int& besti) {
  static_assert(kR == 4, "rows_sum<4>: lane l holds row l / 16");
  if (row0 >= V) return;
  const int nvalid = (int)((V - row0) < kR ? (V - row0) : kR);
  float part[kR];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < kCmax; ++i) a = dot8(w[r][i], xr[i], a);
    part[r] = a;
  }
  // every lane keeps the best of its own row slot; the wave's four slots
  // meet once, after the last rows (lm_head_grid)
  const int r = lane / 16;
  const float y = rbf(rows_sum<kR>(part, lane));
  if (r < nvalid) {
    if ((lane & 15) == 0) logits[row0 + r] = y;
    if (better(y, (int)(row0 + r), best, besti)) {
      best = y;
      besti = (int)(row0 + r);
    }
  }
}

// lm_head over the whole grid with the block's row groups double-buffered in
// registers; publishes the block's (value, index) pick as flag-in-data words.
template <int kCmax, int kR>
__device__ __forceinline__ void lm_head_grid(const u32x4 (&xr)[kCmax], const bf16* __restrict__ W,
                                             float* logits, uint32_t* best_ll, uint32_t tag,
                                             int K, int V, u32x4 (&wa)[kR][kCmax]) {
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
  // the wave's four row slots (lanes 0, 16, 32, 48 hold them)
#pragma unroll
  for (int m = 16; m <= 32; m <<= 1) {
    const float ob = __shfl_xor(best, m, kWave);
    const int oi = __shfl_xor(besti, m, kWave);
    if (better(ob, oi, best, besti)) {
      best = ob;
      besti = oi;
    }
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

// ---------------------------------------------------------------------------
// The kernel (Qwen3-1.7B shape only: H 2048, 16 q / 8 kv heads of 128, I 6144;
// the host entry checks it).
//
// Two roles per XCD, each with its own step loop (one loop holding both
// roles' registers live at once would spill):
//   attention ranks r < 16   the attention (split r of the context when r is
//                            below the step's split count), 8 gate/up rows per
//                            wave, and the down all-reduce (128 rows each)
//   streaming ranks r >= 16  the XCD's qkv rows (8 per wave), 16 gate/up rows
//                            per wave and the down slab requested as soon as
//                            their qkv rows are out -- the rows into registers,
//                            the slab into LDS -- so they stream while the
//                            attention chain runs, when HBM would otherwise
//                            idle; and the o all-reduce (128 rows each)
// Every rank makes 64 rows of the o and down partial products.  Loads retire
// in issue order, so each all-reduce is done by the ranks with no loads in
// flight at that point: the streaming ranks' rows have landed by the o sum,
// and only the streaming ranks request the next layer's qkv rows in front of
// the down sum.  An attention rank requests two of its gate/up rows before
// the scores arithmetic and the rest after its o partials.
//
// A split holds at most kMaxTiles tiles of 64 positions: the context holds at
// most kAttnRanks * kMaxTiles * 64 positions.  Up to three tiles of a split are
// requested at the layer start.
// ---------------------------------------------------------------------------
constexpr int kH = 2048, kQD = 2048, kI = 6144, kD = 128, kG = 2;
constexpr int kXO = kG * kD;                 // 256: an XCD's attention outputs (o's K slice)
constexpr int kXI = kI / kXcds;              // 768: an XCD's intermediate columns (down's K slice)
constexpr int kAttnRanks = 16, kStrmRanks = kRanks - kAttnRanks;
constexpr int kMaxTiles = 8;
constexpr int kRguA = 8, kRguS = 16;         // gate/up rows per wave: attention, streaming ranks
constexpr int kRqkv = 8;                     // qkv rows per wave of a streaming rank
constexpr int kRedRows = kH / kAttnRanks;    // 128: rows each reducer sums
static_assert(kAttnRanks * kRguA + kStrmRanks * kRguS == 2 * kXI / kWavesPerBlock,
              "the roles' gate/up rows cover the XCD's columns");
static_assert(kStrmRanks * kWavesPerBlock * kRqkv == kXO + 2 * kD, "the XCD's q, k and v rows");
static_assert(kAttnRanks == kStrmRanks, "each role's ranks sum an all-reduce's rows");
constexpr int kCH = kH / 512;                // 16-byte chunks per lane of a 2048 row
constexpr int kRhead = 4;
constexpr int kDownLds = 8 * 3 * kWavesPerBlock * kWave;   // u32x4: a streaming rank's down slab

// The block's LDS (declared once in the kernel; both roles use it).
struct XcdLds {
  uint32_t* xs;      // o / down input slice (kXI / 2 words)
  uint32_t* hid_s;   // the hidden state (kH / 2)
  uint32_t* h1_s;    // h1 (kH / 2)
  uint32_t* hs;      // the staged head slice ((kG + 2) * kD / 2)
  float* s_sc;       // the split's scores, G rows of ct * 64
  float* s_new;      // [kG]
  float* red;        // all-reduce staging [kXcds * kRedRows]
  uint32_t* nrm_s;   // the shared input norms (kH / 2)
  u32x4* down;       // a streaming rank's down slab (kDownLds, dynamic)
};

template <bool kAttn>
__device__ __forceinline__ void xcd_steps(const TfdDecodeArgs& a, const TfdXcdArgs& xa, int steps,
                                          int x, int r, const XcdLds& sm) {
  constexpr int kRgu = kAttn ? kRguA : kRguS;
  // attention ranks: gate/up rows requested before the scores arithmetic,
  // which waits on no other block, so they land while it runs
  constexpr int kEarly = kAttn ? 2 : kRgu, kLate = kRgu - kEarly;
  uint32_t* const xs = sm.xs;
  uint32_t* const hid_s = sm.hid_s;
  uint32_t* const h1_s = sm.h1_s;
  uint32_t* const nrm_s = sm.nrm_s;
  const int nb = gridDim.x;
  const int V = a.vocab;
  const float eps = a.eps;
  int* const err = a.err;
  int P = coh_ldi(a.pos);
  int tok = (int)__hip_atomic_load(a.ids, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int lane = threadIdx.x & (kWave - 1);

  // a streaming rank's qkv rows: 32 of XCD x's q (256), k (128) or v (128) rows
  const int sr = r - kAttnRanks;
  const int qkv_row0 = sr < 8 ? kXO * x + 32 * sr
                              : (sr < 12 ? kQD + kD * x + 32 * (sr - 8)
                                         : kQD + 8 * kD + kD * x + 32 * (sr - 12));
  const int vb_qkv = qkv_row0 / (kWavesPerBlock * kRqkv);
  // gate/up rows of XCD x: 2 kXI from row 2 kXI x; the attention ranks' first
  const int vb_gu = kAttn ? (2 * kXI * x) / (kWavesPerBlock * kRgu) + r
                          : (2 * kXI * x + kWavesPerBlock * kAttnRanks * kRguA) /
                                    (kWavesPerBlock * kRgu) + sr;
  // the rows this rank sums in its role's all-reduce (down for attention
  // ranks, o for streaming ranks)
  const int red_q = kAttn ? r : sr;
  const int qkv_n = kQD + 2 * 8 * kD;
  // this XCD's exchange arenas
  uint32_t* const hid_x = word_at(xa.hid, (int64_t)x * (kH / 2));
  uint32_t* const h1_x = word_at(xa.h1, (int64_t)x * (kH / 2));
  const int64_t heads_words = (int64_t)a.nsplit * (kXcds * kG);
  uint32_t* const smax_x = word_at(xa.smax, x * heads_words);
  uint32_t* const psum_x = word_at(xa.psum, x * heads_words);
  uint32_t* const pout_x = word_at(xa.pout, x * heads_words * kD);
  uint32_t* const attn_x = word_at(a.x_attn, (int64_t)x * (kXO / 2));   // the merged outputs
  uint32_t* const mid_x = word_at(a.x_mid, (int64_t)x * (kXI / 2));     // the SwiGLU values
  uint32_t* const opart_x = word_at(xa.opart, (int64_t)x * kH);
  uint32_t* const dpart_x = word_at(xa.dpart, (int64_t)x * kH);

  u32x4 we[kEarly][kCH], wo[8][1], wd[8][3];
  u32x4 wl[kLate > 0 ? kLate : 1][kCH];
  u32x4 wq[kAttn ? 1 : kRqkv][kCH];
  u32x4 gq_in[kCH], gq_post[kCH];
  if constexpr (!kAttn) {
    gemv_issue<kCH, kRqkv>(vb_qkv, (const bf16*)a.layers[0].w_qkv, kH, qkv_n, wq);
    load_x<kCH>((const bf16*)a.layers[0].gamma_in, kH / 8, lane, gq_in);
  }
  // the layer table's entry for the next layer is read a layer ahead, so no
  // layer's first loads wait on the read of their addresses
  TfdLayer wn = a.layers[0];
  for (int t = 0; t < steps; ++t, ++P) {
    uint64_t* tl = (a.timeline && t < a.timeline_steps)
                       ? a.timeline + ((int64_t)t * nb + blockIdx.x) * (14 * a.n_layers + 4)
                       : nullptr;
    const uint32_t tag0 = a.epoch + (uint32_t)t * (uint32_t)(a.n_layers + 1);
    {
      const int id = (tok >= 0 && tok < V) ? tok : 0;
      const uint32_t* row = reinterpret_cast<const uint32_t*>((const bf16*)a.w_embed +
                                                              (int64_t)id * kH);
      for (int i = threadIdx.x; i < kH / 8; i += kBlock)
        *reinterpret_cast<u32x4*>(hid_s + 4 * i) = *reinterpret_cast<const u32x4*>(row + 4 * i);
    }
    const int Pc = (P >= 0 && P < a.max_pages * kPage) ? P : 0;
    // the prior context in at most kAttnRanks splits of ct tiles; rank r <
    // parts owns split r (the host bounds the context so ct <= kMaxTiles)
    const int ntile = (Pc + kSplit - 1) / kSplit;
    const int ct = ntile > kAttnRanks ? (ntile + kAttnRanks - 1) / kAttnRanks : 1;
    const int slen = ct * kSplit;
    const int nact = (Pc + slen - 1) / slen;
    const int parts = nact > 0 ? nact : 1;
    // what the first three K / V tiles and the q/k operands read depends on
    // the position only: the pages, the rope rows and the new position's page
    // are looked up once per step, so no layer's tile addresses wait on a
    // load.  A split's tiles past its last are its first again: those loads
    // hit the lines the first brought into the L2, and loads that are always
    // issued keep every later wait count exact.
    const int s0 = r < parts ? r : parts;
    const int j0 = s0 * slen, j1 = ct > 1 ? j0 + kSplit : j0, j2 = ct > 2 ? j0 + 2 * kSplit : j0;
    KTile<kD> kt0, kt1p, kt2p;
    VTile<kD> vt0, vt1p, vt2p;
    QKPre pre0{};
    if constexpr (kAttn) {
      k_tile_pages<kD>(j0, a.page_table, a.max_pages, kt0);
      v_tile_pages<kD>(j0, a.page_table, a.max_pages, vt0);
      k_tile_pages<kD>(j1, a.page_table, a.max_pages, kt1p);
      v_tile_pages<kD>(j1, a.page_table, a.max_pages, vt1p);
      k_tile_pages<kD>(j2, a.page_table, a.max_pages, kt2p);
      v_tile_pages<kD>(j2, a.page_table, a.max_pages, vt2p);
      pre0 = qk_prefetch<kD, kG>(P, P, (const bf16*)a.layers[0].gamma_q,
                                 (const bf16*)a.layers[0].gamma_k, (const bf16*)a.cos_table,
                                 (const bf16*)a.sin_table, a.rope_rows, a.page_table,
                                 a.max_pages);
    }
    __syncthreads();
    for (int l = 0; l < a.n_layers; ++l) {
      const TfdLayer w = wn;
      wn = a.layers[(l + 1) % a.n_layers];
      const uint32_t tag = tag0 + (uint32_t)l + 1u;
      const bool last = l + 1 == a.n_layers;
      stamp(tl);
      if constexpr (kAttn) {
        // the split's first K / V tiles, the q/k norm scales and the o slab
        // depend on no other block: requested first, they land while the
        // streaming ranks make the QKV projection.  The tiles load
        // unconditionally (a tile past P reads valid rows the attention
        // masks): loads under a branch make a later wait also wait for them.
        KTile<kD> kt, kt1, kt2;
        VTile<kD> vt, vt1, vt2;
        QKPre pre = pre0;
#pragma unroll
        for (int p = 0; p < AttnShape<kD>::kKPasses; ++p) {
          kt.pg[p] = kt0.pg[p];
          kt1.pg[p] = kt1p.pg[p];
          kt2.pg[p] = kt2p.pg[p];
        }
#pragma unroll
        for (int p = 0; p < AttnShape<kD>::kVPasses; ++p) {
          vt.pg[p] = vt0.pg[p];
          vt1.pg[p] = vt1p.pg[p];
          vt2.pg[p] = vt2p.pg[p];
        }
        k_tile_load_pages<kD, true>(j0, x, (const bf16*)w.k_pool, a.num_pages, 8, kt);
        v_tile_load_pages<kD, true>(j0, x, (const bf16*)w.v_pool, a.num_pages, 8, vt);
        k_tile_load_pages<kD, true>(j1, x, (const bf16*)w.k_pool, a.num_pages, 8, kt1);
        v_tile_load_pages<kD, true>(j1, x, (const bf16*)w.v_pool, a.num_pages, 8, vt1);
        k_tile_load_pages<kD, true>(j2, x, (const bf16*)w.k_pool, a.num_pages, 8, kt2);
        v_tile_load_pages<kD, true>(j2, x, (const bf16*)w.v_pool, a.num_pages, 8, vt2);
        qk_gammas<kD, kG>((const bf16*)w.gamma_q, (const bf16*)w.gamma_k, pre);
        slab_issue<1>((const bf16*)w.w_o, kQD, 64 * r, kXO * x, wo);
        stamp(tl);
        if (r >= parts) {
          rows_issue<kCH, kRgu, kEarly>(vb_gu, (const bf16*)w.w_gu, kH, 0, we);
          stamp(tl); stamp(tl); stamp(tl); stamp(tl); stamp(tl); stamp(tl);
        } else {
          const AttnLL ll{a.x_qkv, smax_x, psum_x, pout_x, a.x_attn, tag};
          // ---- attention part 1: scores over split r of kv head x
          stage_head_ll<kD, kG, kXcdLocal>(x, 8 * kG, 8, ll, sm.hs, err);
          __syncthreads();
          rows_issue<kCH, kRgu, kEarly>(vb_gu, (const bf16*)w.w_gu, kH, 0, we);
          stamp(tl);
          attn_scores_phase<kD, kG, true, kXcdLocal, BlockGrp, true>(r, x, sm.hs, pre, a.rope_rows, P, P,
                                                     a.page_table, a.max_pages, (bf16*)w.k_pool,
                                                     (bf16*)w.v_pool, a.num_pages, 8, a.scale,
                                                     eps, sm.s_sc, 0, nullptr, sm.s_new, ll, kt,
                                                     err, ct, &kt1, &kt2);
          stamp(tl);
          // ---- part 2: P.V partials
          stamp(tl);
          attn_pv_phase<kD, kG, true, NoHook, RowOut, kXcdLocal, BlockGrp, true>(
              r, x, a.nsplit, nullptr, P, a.page_table, a.max_pages, (const bf16*)w.v_pool,
              a.num_pages, 8, sm.s_sc, 0, nullptr, sm.s_new, nullptr, nullptr, nullptr, nullptr,
              ll, vt, err, ct, NoHook{}, RowOut{}, &vt1, &vt2);
          stamp(tl);
          // ---- part 3: merge
          stamp(tl);
          attn_merge_ll<kD, kG, NoHook, kXcdLocal>(r, x, P, a.max_pages, 8, sm.s_new, ll, err,
                                                   NoHook{}, ct);
          __syncthreads();
          stamp(tl);
        }
      } else {
        slab_issue<1>((const bf16*)w.w_o, kQD, 64 * r, kXO * x, wo);
        // ---- qkv (the hidden state is in hid_s)
        gemv_finish_ll<kCH, kRqkv, kNorm, kStore, kXcdLocal>(vb_qkv, hid_s, gq_in, nullptr,
                                                             a.x_qkv, tag, kH, qkv_n, eps, wq,
                                                             nrm_s);
        stamp(tl);
        // every gate/up row and the down slab: they land during the attention
        rows_issue<kCH, kRgu, kEarly>(vb_gu, (const bf16*)w.w_gu, kH, 0, we);
        slab_to_lds<3>((const bf16*)w.w_down, kI, 64 * r, kXI * x, sm.down);
        stamp(tl); stamp(tl); stamp(tl); stamp(tl); stamp(tl); stamp(tl);
      }
      // ---- o: this XCD's 256 attention outputs against the o slab
      ll_stage<kXcdLocal>(attn_x, kXO, tag, xs, err);
      __syncthreads();
      stamp(tl);
      slab_finish<1>(xs, wo, opart_x, 64 * r, tag);
      stamp(tl);
      if constexpr (kAttn) {
        // the remaining gate/up rows stream while the streaming ranks sum o
        rows_issue<kCH, kRgu, kLate>(vb_gu, (const bf16*)w.w_gu, kH, kEarly, wl);
        load_x<kCH>((const bf16*)w.gamma_post, kH / 8, lane, gq_post);
      } else {
        load_x<kCH>((const bf16*)w.gamma_post, kH / 8, lane, gq_post);
        allreduce_publish<kRedRows>(xa.opart, kH, red_q, hid_s, h1_x, tag, sm.red, err);
      }
      ll_stage<kXcdLocal>(h1_x, kH, tag, h1_s, err);
      __syncthreads();
      stamp(tl);
      // ---- gate/up + SwiGLU: this block's share of the XCD's 768 columns
      {
        u32x4 wg[kRgu][kCH];
#pragma unroll
        for (int i = 0; i < kRgu; ++i)
#pragma unroll
          for (int c = 0; c < kCH; ++c)
            wg[i][c] = i < kEarly ? we[i][c] : wl[(i - kEarly) % (kLate > 0 ? kLate : 1)][c];
        gemv_finish_ll<kCH, kRgu, kNorm, kSwiglu, kXcdLocal>(vb_gu, h1_s, gq_post, nullptr,
                                                             a.x_mid, tag, kH, 2 * kI, eps, wg,
                                                             nrm_s);
      }
      stamp(tl);
      if constexpr (kAttn) slab_issue<3>((const bf16*)w.w_down, kI, 64 * r, kXI * x, wd);
      // ---- down: this XCD's 768 SwiGLU values against the down slab
      ll_stage<kXcdLocal>(mid_x, kXI, tag, xs, err);
      __syncthreads();
      stamp(tl);
      if constexpr (!kAttn) slab_from_lds<3>(sm.down, wd);
      slab_finish<3>(xs, wd, dpart_x, 64 * r, tag);
      if constexpr (kAttn) {
        allreduce_publish<kRedRows>(xa.dpart, kH, red_q, h1_s, hid_x, tag, sm.red, err);
        // the layer output is the next layer's input only for the streaming
        // ranks (the qkv rows); an attention rank reads it for the head
        if (last) {
          ll_stage<kXcdLocal>(hid_x, kH, tag, hid_s, err);
          __syncthreads();
        }
      } else {
        // the next layer's qkv weights -- after the last layer, layer 0's for
        // the next step -- stream while the attention ranks sum down
        gemv_issue<kCH, kRqkv>(vb_qkv, (const bf16*)wn.w_qkv, kH, qkv_n, wq);
        load_x<kCH>((const bf16*)wn.gamma_in, kH / 8, lane, gq_in);
        ll_stage<kXcdLocal>(hid_x, kH, tag, hid_s, err);
        __syncthreads();
      }
      stamp(tl);
    }
    // ---- head: final norm, logits, block pick
    {
      const uint32_t tag_head = tag0 + (uint32_t)a.n_layers;
      u32x4 wa[kRhead][kCH], gr[kCH];
      gemv_issue<kCH, kRhead>((int)blockIdx.x, (const bf16*)a.w_head, kH, V, wa);
      load_x<kCH>((const bf16*)a.gamma_final, kH / 8, lane, gr);
      stamp(tl);
      u32x4 xr[kCH];
      x_from_lds<kCH>(hid_s, kH / 8, lane, xr);
      rms_norm_apply<kCH>(xr, gr, kH, eps);
      lm_head_grid<kCH, kRhead>(xr, (const bf16*)a.w_head, a.logits, a.x_best, tag_head + 1u, kH,
                                V, wa);
      stamp(tl);
    }
    stamp(tl);
    tok = finalize_ll(a.x_best, nb, tag0 + (uint32_t)a.n_layers + 1u, P, a.inp, a.prompt_len,
                      a.nsteps, V, a.ids, a.pos, a.sam, err);
    stamp(tl);
    if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSync) break;
  }
}

__global__ __launch_bounds__(kBlock) void k_decode_xcd(TfdDecodeArgs a, TfdXcdArgs xa, int steps) {
  __shared__ __attribute__((aligned(16))) uint32_t xs[kXI / 2];
  __shared__ __attribute__((aligned(16))) uint32_t hid_s[kH / 2];
  __shared__ __attribute__((aligned(16))) uint32_t h1_s[kH / 2];
  __shared__ __attribute__((aligned(16))) uint32_t hs[(kG + 2) * kD / 2];
  __shared__ float s_sc[kG * kMaxTiles * kSplit];
  __shared__ float s_new[kG];
  __shared__ float red[kXcds * kRedRows];
  __shared__ __attribute__((aligned(16))) uint32_t nrm_s[kH / 2];
  extern __shared__ __attribute__((aligned(16))) u32x4 dyn_lds[];   // kDownLds
  const int xcc = xcc_id();
  const int x = xcc & (kXcds - 1), r = (int)blockIdx.x / kXcds;
  if (threadIdx.x == 0 && xcc != x) raise_error(a.err, kErrPlacement | kErrSync);
  const XcdLds sm{xs, hid_s, h1_s, hs, s_sc, s_new, red, nrm_s, dyn_lds};
  if (r < kAttnRanks)
    xcd_steps<true>(a, xa, steps, x, r, sm);
  else
    xcd_steps<false>(a, xa, steps, x, r, sm);
}

}  // namespace

extern "C" {

int tfd_decode_xcd(const TfdDecodeArgs* args, const TfdXcdArgs* xcd, int steps, void* stream) {
  if (!args || !xcd) return fail(kBadArg, "decode_xcd: null args");
  const TfdDecodeArgs& a = *args;
  const TfdXcdArgs& xa = *xcd;
  if (!a.layers || !a.w_embed || !a.w_head || !a.gamma_final || !a.cos_table || !a.sin_table ||
      !a.page_table || !a.x_qkv || !a.x_attn || !a.x_mid || !a.x_best || !a.logits || !a.ids ||
      !a.pos || !a.inp || !a.prompt_len || !a.sam || !a.err || !xa.hid || !xa.h1 || !xa.opart ||
      !xa.dpart || !xa.smax || !xa.psum || !xa.pout)
    return fail(kBadArg, "decode_xcd: null pointer in args");
  if (steps < 0) return fail(kBadArg, "decode_xcd: steps=%d", steps);
  if (steps == 0) return 0;
  if (a.n_layers <= 0 || a.hidden != kH || a.heads != 16 || a.kv_heads != 8 ||
      a.head_dim != kD || a.intermediate != kI || a.vocab <= 0 || a.nsteps <= 0)
    return fail(kUnsupported,
                "decode_xcd: partitioned for hidden 2048, 16 q / 8 kv heads of 128, "
                "intermediate 6144 (got %d, %d / %d of %d, %d)",
                a.hidden, a.heads, a.kv_heads, a.head_dim, a.intermediate);
  if ((uint64_t)a.epoch + (uint64_t)steps * (uint64_t)(a.n_layers + 1) >= 0xffffffffull)
    return fail(kBadArg, "decode_xcd: epoch %u + %d steps passes 2^32: zero the exchange "
                "buffers and restart the epoch at 0", a.epoch, steps);
  if ((int64_t)a.nsplit * kSplit < (int64_t)a.max_pages * kPage || a.num_pages <= 0 ||
      a.nsplit > kAttnRanks * kMaxTiles)
    return fail(kBadShape, "decode_xcd: nsplit=%d must cover max_pages=%d and be at most %d",
                a.nsplit, a.max_pages, kAttnRanks * kMaxTiles);
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return fail((int)e, "decode_xcd: device query failed");
  const int grid = kXcds * kRanks;
  if (cus != grid)
    return fail(kUnsupported, "decode_xcd: needs %d compute units (8 XCDs of 32), device has %d",
                grid, cus);
  int per_cu = 0;
  const void* fn = reinterpret_cast<const void*>(&k_decode_xcd);
  const size_t dyn = kDownLds * sizeof(u32x4);
  // the dynamic-LDS attribute is set once per device (with that device current)
  static bool lds_set[64] = {};
  if (dev < 0 || dev >= 64) return fail(kUnsupported, "decode_xcd: device %d", dev);
  if (!lds_set[dev]) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn);
    if (e != hipSuccess)
      return fail((int)e, "decode_xcd: %zu bytes of dynamic LDS refused", dyn);
    lds_set[dev] = true;
  }
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kBlock, dyn);
  if (e != hipSuccess) return fail((int)e, "decode_xcd: occupancy query failed");
  if (per_cu < 1)
    return fail(kUnsupported, "decode_xcd: a block does not fit a compute unit");
  TfdDecodeArgs karg = a;
  TfdXcdArgs kx = xa;
  int ksteps = steps;
  void* kargs[] = {&karg, &kx, &ksteps};
  static const bool plain = [] {
    const char* v = getenv("TFD_PLAIN_LAUNCH");
    return v && v[0] == '1';
  }();
  if (plain)
    e = hipLaunchKernel(fn, dim3(grid), dim3(kBlock), kargs, dyn, (hipStream_t)stream);
  else
    e = hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kBlock), kargs, (unsigned)dyn,
                                   (hipStream_t)stream);
  if (e != hipSuccess) return fail((int)e, "decode_xcd: launch failed: %s", hipGetErrorString(e));
  return launched("decode_xcd");
}

}  // extern "C"
