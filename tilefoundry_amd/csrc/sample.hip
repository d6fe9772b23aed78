// Sampling a token per row of f32 logits, on the device, for gfx950.
//
// The reference's runtimes choose a token two ways besides argmax:
//   * top-k first, then temperature, softmax over the k, the top-p nucleus
//     inside them, a categorical draw (examples/qwen3_5_35b_a3b-tilelang/
//     run.py:145-180, on the host with torch);
//   * softmax(logits / T) over the whole vocabulary by Gumbel-max inside the
//     captured step (examples/granite_4_0_h_small-cuda/kernels/granite.cu:
//     716-800).
// Both are here as one entry, tfd_sample_rows: top_k in 1..TFD_SAMPLE_MAX_K takes
// the first way, top_k = 0 (with top_p = 1) the second.  Either way the random
// numbers come from a counter-based hash of (seed, row, counter[row], element)
// -- the engines pass each row's position as its counter -- so a step captured
// in a HIP graph draws new numbers on every replay and a run is reproducible
// from its seed.  The streams are this library's own (the reference's torch
// generator and Philox streams are not reproduced): a sampled stream is checked
// by distribution and against the CPU restatement given the same uniforms, not
// token for token against the reference.
//
// Top-k.  Logit i's key is (its value's order bits << 32) | (2^32 - 1 - i):
// unique, larger for a larger value and, among equal values, for the lower
// index (the argmax rule); NaN ranks below every number and -0 as +0.  Stage 1:
// each wave takes 1024 logits (16 per lane) and extracts its k largest keys in
// k rounds (a wave max of the lanes' bests; the winning lane drops the key and
// rescans its 16).  Stage 2, one block per row: each of 16 waves merges its
// share of the chunks' candidates the same way, then one wave merges the 16
// lists; the k keys come out in descending order.  One thread then applies
// temperature, softmax, top-p and the draw in index order, as run.py does.

#include "decode_phases.h"
#include "host_common.h"
#include "tf_decode.h"

using namespace tfd;
using namespace tfd_host;

namespace {

constexpr int kMaxK = TFD_SAMPLE_MAX_K;
constexpr int kChunk = 1024;                    // logits per stage-1 wave
constexpr int kPerLane = kChunk / kWave;        // 16
constexpr int kMaxChunks = 16 * kPerLane;       // stage 2: 16 waves x 16 chunk lists each
constexpr int kGumbelChunks = 64;               // blocks per row of the Gumbel path

// splitmix64's output function (Steele, Lea and Flood, "Fast splittable
// pseudorandom number generators", OOPSLA 2014): a bijective 64-bit mix.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
// 24 random bits of (seed, row, counter, element): the hash of the hash chain
__device__ __forceinline__ uint32_t rand24(uint64_t seed, int row, int ctr, uint32_t elem) {
  const uint64_t h = mix64(mix64(mix64(seed) + (uint64_t)(uint32_t)row) +
                           (((uint64_t)(uint32_t)ctr << 32) | elem));
  return (uint32_t)(h >> 40);
}
constexpr uint32_t kDrawElem = 0xffffffffu;     // the element id of a row's top-k draw

__device__ __forceinline__ uint64_t logit_key(float v, int i) {
  uint32_t b = __float_as_uint(v);
  uint32_t ord;
  if ((b & 0x7fffffffu) > 0x7f800000u) {
    ord = 0;                                    // NaN: below every number
  } else {
    if (b == 0x80000000u) b = 0;                // -0 ranks as +0
    ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
}
__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t ord = (uint32_t)(key >> 32);
  if (ord == 0) return __uint_as_float(0x7fc00000u);
  return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}
__device__ __forceinline__ int key_index(uint64_t key) {
  return (int)(0xffffffffu - (uint32_t)key);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m, kWave);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, kWave);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

// The k largest of a wave's keys (kN per lane; 0 = no key), in descending
// order, to out[0..k) by lane 0 (keys that run out leave 0).
template <int kN>
__device__ __forceinline__ void wave_topk(uint64_t (&key)[kN], int k, uint64_t* out) {
  const int lane = threadIdx.x & (kWave - 1);
  uint64_t best = 0;
#pragma unroll
  for (int j = 0; j < kN; ++j) best = key[j] > best ? key[j] : best;
  for (int r = 0; r < k; ++r) {
    const uint64_t w = wave_max_u64(best);
    if (lane == 0) out[r] = w;
    if (w != 0 && best == w) {                  // keys are unique: one lane owns it
      best = 0;
#pragma unroll
      for (int j = 0; j < kN; ++j) {
        if (key[j] == w) key[j] = 0;
        best = key[j] > best ? key[j] : best;
      }
    }
  }
}

// stage 1: wave c of row `row` -> work[row][c][0..k)
__global__ __launch_bounds__(kBlock) void k_sample_topk_part(const float* __restrict__ logits,
                                                             int ldl, int V, int k,
                                                             uint64_t* __restrict__ work,
                                                             int nchunk) {
  const int row = blockIdx.y, lane = threadIdx.x & (kWave - 1);
  const int c = blockIdx.x * kWavesPerBlock + (int)threadIdx.x / kWave;
  if (c >= nchunk) return;
  const float* r = logits + (int64_t)row * ldl;
  uint64_t key[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int i = c * kChunk + j * kWave + lane;
    key[j] = i < V ? logit_key(r[i], i) : 0;
  }
  wave_topk<kPerLane>(key, k, work + ((int64_t)row * nchunk + c) * k);
}

// stage 2: one block of 16 waves per row
__global__ __launch_bounds__(1024) void k_sample_topk_pick(
    const uint64_t* __restrict__ work, int nchunk, int k, float temperature, float top_p,
    uint64_t seed, const int* __restrict__ ctr, int* __restrict__ pick) {
  const int row = blockIdx.x, lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  __shared__ uint64_t lists[16][kMaxK];
  __shared__ uint64_t top[kMaxK];
  __shared__ float x[kMaxK];
  const uint64_t* w = work + (int64_t)row * nchunk * k;
  {
    // wave `wave` merges chunks wave, wave + 16, ...: at most 16 lists of k
    uint64_t key[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int slot = j * kWave + lane;        // slot / k: list, slot % k: rank
      const int c = wave + 16 * (slot / k);
      key[j] = (slot / k < 16 && c < nchunk && slot < 16 * k) ? w[(int64_t)c * k + slot % k] : 0;
    }
    wave_topk<kPerLane>(key, k, lists[wave]);
  }
  __syncthreads();
  if (wave == 0) {
    uint64_t key[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int slot = j * kWave + lane;
      key[j] = slot < 16 * k ? lists[slot / k][slot % k] : 0;
    }
    wave_topk<kPerLane>(key, k, top);
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  // temperature, softmax over the k, the nucleus, the draw (run.py:166-179),
  // in index order; a NaN candidate (fewer than k numbers in the row) weighs 0
  int n = 0;
  while (n < k && top[n] != 0) ++n;
  int choice = n > 0 ? key_index(top[0]) : 0;
  for (int i = 0; i < n; ++i) {
    const float v = key_value(top[i]);
    x[i] = temperature != 1.0f ? v / temperature : v;
  }
  const float m = n > 0 ? x[0] : 0.f;
  float s = 0.f;
  for (int i = 0; i < n; ++i) {
    x[i] = x[i] == x[i] ? expf(x[i] - m) : 0.f;
    s += x[i];
  }
  if (n > 0 && s > 0.f && s == s) {
    float kept = 0.f, before = 0.f;
    int last = 0;
    for (int i = 0; i < n; ++i) {
      const float p = x[i] / s;
      const bool keep = i == 0 || top_p >= 1.0f || before < top_p;
      before += p;
      x[i] = keep ? p : 0.f;
      if (keep) {
        kept += p;
        last = i;
      }
    }
    const float u = (float)rand24(seed, row, ctr ? ctr[row] : 0, kDrawElem) * (1.0f / 16777216.0f);
    const float target = u * kept;
    float acc = 0.f;
    int at = last;
    for (int i = 0; i <= last; ++i) {
      acc += x[i];
      if (x[i] > 0.f && target < acc) {
        at = i;
        break;
      }
    }
    choice = key_index(top[at]);
  }
  pick[row] = choice;
}

// Gumbel-max: chunk winners of v / T - log(-log(u)), u in (0, 1), the lower
// index on ties; a NaN never wins (an all-NaN row picks 0)
__global__ __launch_bounds__(kBlock) void k_sample_gumbel_part(const float* __restrict__ logits,
                                                               int ldl, int V, float temperature,
                                                               uint64_t seed,
                                                               const int* __restrict__ ctr,
                                                               int* __restrict__ part) {
  const int row = blockIdx.y, chunk = blockIdx.x;
  const int per = (V + kGumbelChunks - 1) / kGumbelChunks;
  const int k0 = chunk * per, k1 = k0 + per < V ? k0 + per : V;
  const float* r = logits + (int64_t)row * ldl;
  const int c = ctr ? ctr[row] : 0;
  float b = kNegInf;
  int bi = 0x7fffffff;
  for (int i = k0 + (int)threadIdx.x; i < k1; i += kBlock) {
    // 23 bits: (b + 0.5) * 2^-23 is exact in f32, so u stays inside (0, 1)
    const float u = ((float)(rand24(seed, row, c, (uint32_t)i) >> 1) + 0.5f) *
                    (1.0f / 8388608.0f);
    const float v = r[i];
    const float g = (temperature != 1.0f ? v / temperature : v) - logf(-logf(u));
    if (better(g, i, b, bi)) {
      b = g;
      bi = i;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ob = __shfl_xor(b, m, kWave);
    const int oi = __shfl_xor(bi, m, kWave);
    if (better(ob, oi, b, bi)) {
      b = ob;
      bi = oi;
    }
  }
  __shared__ float sv[kWavesPerBlock];
  __shared__ int si[kWavesPerBlock];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = b;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWavesPerBlock; ++w)
      if (better(sv[w], si[w], b, bi)) {
        b = sv[w];
        bi = si[w];
      }
    part[((int64_t)row * kGumbelChunks + chunk) * 2] = __float_as_int(b);
    part[((int64_t)row * kGumbelChunks + chunk) * 2 + 1] = bi;
  }
}

__global__ __launch_bounds__(kWave) void k_sample_gumbel_pick(const int* __restrict__ part,
                                                              int V, int* __restrict__ pick) {
  const int row = blockIdx.x, lane = threadIdx.x;
  float b = __int_as_float(part[((int64_t)row * kGumbelChunks + lane) * 2]);
  int i = part[((int64_t)row * kGumbelChunks + lane) * 2 + 1];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ob = __shfl_xor(b, m, kWave);
    const int oi = __shfl_xor(i, m, kWave);
    if (better(ob, oi, b, i)) {
      b = ob;
      i = oi;
    }
  }
  if (lane == 0) pick[row] = (i >= 0 && i < V) ? i : 0;
}

static_assert(kGumbelChunks == kWave, "one chunk winner per lane of the pick");

}  // namespace

extern "C" {

int64_t tfd_sample_work_bytes(int rows, int vocab, int top_k) {
  if (rows <= 0 || vocab <= 0 || top_k < 0 || top_k > kMaxK) return -1;
  if (top_k == 0) return (int64_t)rows * kGumbelChunks * 2 * (int64_t)sizeof(int32_t);
  const int64_t nchunk = (vocab + kChunk - 1) / kChunk;
  return (int64_t)rows * nchunk * top_k * (int64_t)sizeof(uint64_t);
}

int tfd_sample_rows(const float* logits, int ldl, int rows, int vocab,
                    const TfdSampling* sampling, const int32_t* counter, int32_t* pick,
                    void* work, int64_t work_bytes, void* stream) {
  if (!logits || !sampling || !pick || !work) return fail(kBadArg, "sample_rows: null pointer");
  const TfdSampling& sp = *sampling;
  if (rows <= 0 || rows > 65535 || vocab <= 0 || ldl < vocab || vocab > TFD_SAMPLE_MAX_VOCAB)
    return fail(kBadShape, "sample_rows: rows=%d vocab=%d ldl=%d (vocab at most %d)", rows,
                vocab, ldl, TFD_SAMPLE_MAX_VOCAB);
  if (!(sp.temperature > 0.f) || !(sp.top_p > 0.f && sp.top_p <= 1.f) || sp.top_k < 0 ||
      sp.top_k > kMaxK)
    return fail(kBadArg, "sample_rows: temperature=%g top_k=%d top_p=%g (temperature > 0, "
                "top_k 0..%d, top_p in (0, 1])", sp.temperature, sp.top_k, sp.top_p, kMaxK);
  if (sp.top_k == 0 && sp.top_p < 1.f)
    return fail(kBadArg, "sample_rows: top_p=%g needs top_k >= 1 (the nucleus is taken "
                "inside the top k)", sp.top_p);
  const int64_t need = tfd_sample_work_bytes(rows, vocab, sp.top_k);
  if (work_bytes < need)
    return fail(kBadShape, "sample_rows: work of %lld bytes, %lld needed", (long long)work_bytes,
                (long long)need);
  auto s = (hipStream_t)stream;
  if (sp.top_k == 0) {
    hipLaunchKernelGGL(k_sample_gumbel_part, dim3(kGumbelChunks, rows), dim3(kBlock), 0, s,
                       logits, ldl, vocab, sp.temperature, sp.seed, counter, (int*)work);
    hipLaunchKernelGGL(k_sample_gumbel_pick, dim3(rows), dim3(kWave), 0, s, (const int*)work,
                       vocab, pick);
    return launched("sample_rows");
  }
  const int nchunk = (vocab + kChunk - 1) / kChunk;
  static_assert(kMaxChunks * kChunk >= TFD_SAMPLE_MAX_VOCAB, "stage 2 holds every chunk list");
  hipLaunchKernelGGL(k_sample_topk_part,
                     dim3((nchunk + kWavesPerBlock - 1) / kWavesPerBlock, rows), dim3(kBlock), 0,
                     s, logits, ldl, vocab, sp.top_k, (uint64_t*)work, nchunk);
  hipLaunchKernelGGL(k_sample_topk_pick, dim3(rows), dim3(1024), 0, s, (const uint64_t*)work,
                     nchunk, sp.top_k, sp.temperature, sp.top_p, sp.seed, counter, pick);
  return launched("sample_rows");
}

}  // extern "C"
