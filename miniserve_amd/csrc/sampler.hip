// Temperature / top-k / top-p sampling without a vocabulary sort (runner/sampler.py of the
// reference: apply_top_k_top_p, compute_probs, sample).
//
// One workgroup of 1024 threads per row; the row's logits stay in global memory (L2 / Infinity
// Cache) and are re-read by each pass:
//  1. z = logits / temperature (IEEE division, as `logits / temps`), the row maximum m, and for a
//     greedy row the first index of the largest raw logit (`logits.argmax`).
//  2. top-k (0 < k < vocab): the k-th largest z by radix select over order-preserving 32-bit keys,
//     four 8-bit digits, integer counts in LDS. Every z >= that value is kept (the reference masks
//     `sorted < kth`).
//  3. top-p (p < 1): the reference sorts the kept logits ascending, takes the cumulative softmax
//     and drops every token whose cumulative probability is <= 1 - p (never the largest). The same
//     cut is found by a radix select on probability mass: the smallest key whose mass at or below
//     it exceeds (1 - p), with each token's mass exp(z - m) / Z in 2^-44 fixed point and 64-bit
//     integer sums (exact, order-free). Tokens of equal value are kept or dropped together.
//  4. One output pass over the kept set K, with Z_K = sum over K of exp(z - m):
//     MASK   out = z on K, -inf elsewhere            (apply_top_k_top_p; temperature 1)
//     PROBS  out = exp(z - m) / Z_K on K, 0 elsewhere  (compute_probs)
//     SAMPLE id  = first argmax over K of (exp(z - m) / Z_K) / noise  (the exponential race of
//            `sample`, noise ~ Exp(1) supplied by the caller), or the greedy id.
// Float sums (Z) are per-thread in a fixed order, then a fixed tree: deterministic.
#include <hip/hip_runtime.h>

#include "common.h"

namespace msa {

constexpr int kSampThreads = 1024;
constexpr int kSampWaves = kSampThreads / 64;
constexpr double kMassScale = 17592186044416.0;  // 2^44: mass fixed point (sum of <= 2^31 values < 2^64)

enum SampMode { SAMP_MASK = 0, SAMP_PROBS = 1, SAMP_SAMPLE = 2 };

struct SampArgs {
  const float* logits;
  int64_t ld;
  int64_t vocab;
  const float* temperature;  // null: 1
  const int32_t* top_k;      // null or k outside (0, vocab): no top-k
  const float* top_p;        // null or p >= 1: no top-p
  const uint8_t* greedy;     // SAMPLE: nonzero rows take the greedy id
  const float* noise;        // SAMPLE: [rows][ldn]
  int64_t ldn;
  float* out;  // MASK / PROBS: [rows][ldo]
  int64_t ldo;
  int64_t* ids;  // SAMPLE: [rows]
  int mode;
};

// Order-preserving key: unsigned comparison of keys = float comparison (finite values, +-inf).
__device__ __forceinline__ uint32_t ord_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct SampShared {
  union {
    uint32_t cnt[256];
    unsigned long long mass[256];
  } hist;
  float fred[kSampWaves];
  int ired[kSampWaves];
  uint32_t bcast_u[2];
  unsigned long long bcast_ull;
};

__device__ __forceinline__ float block_max(float v, SampShared& sh) {
  v = fmaxf(v, __shfl_xor(v, 1));
  v = fmaxf(v, __shfl_xor(v, 2));
  v = fmaxf(v, __shfl_xor(v, 4));
  v = fmaxf(v, __shfl_xor(v, 8));
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh.fred[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = fmaxf(r, sh.fred[w]);
  return r;
}

__device__ __forceinline__ float block_sum(float v, SampShared& sh) {
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) r += sh.fred[w];  // fixed order
  return r;
}

// First index of the largest value: (v, i) pairs, larger v wins, equal v -> smaller i.
__device__ __forceinline__ int block_argmax(float v, int i, SampShared& sh) {
  for (int off = 1; off < 64; off <<= 1) {
    const float ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(i, off);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    sh.fred[threadIdx.x >> 6] = v;
    sh.ired[threadIdx.x >> 6] = i;
  }
  __syncthreads();
  float bv = sh.fred[0];
  int bi = sh.ired[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
    if (sh.fred[w] > bv || (sh.fred[w] == bv && sh.ired[w] < bi)) {
      bv = sh.fred[w];
      bi = sh.ired[w];
    }
  return bi;
}

// The whole row in one workgroup (kSampThreads threads; MASK, PROBS, and SAMPLE rows the
// chunked path below does not take).
__device__ void sample_row(const SampArgs& a, int64_t row, SampShared& sh) {
  const int nt = blockDim.x;  // any multiple of 64 up to nt
  const float* lg = a.logits + row * a.ld;
  const int64_t V = a.vocab;
  const int tid = threadIdx.x;

  if (a.mode == SAMP_SAMPLE && a.greedy && a.greedy[row]) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int64_t i = tid; i < V; i += nt) {
      const float v = lg[i];
      if (v > bv) {  // ascending i: the first of equal maxima stays
        bv = v;
        bi = (int)i;
      }
    }
    const int id = block_argmax(bv, bi, sh);
    if (tid == 0) a.ids[row] = id == 0x7fffffff ? 0 : id;  // a row of -inf: index 0, as argmax
    return;
  }

  const float t = a.temperature ? a.temperature[row] : 1.0f;
  float mloc = -INFINITY;
  for (int64_t i = tid; i < V; i += nt) mloc = fmaxf(mloc, lg[i] / t);
  const float m = block_max(mloc, sh);

  // ---- top-k: key of the k-th largest z -----------------------------------------------------
  uint32_t kmin = 0;  // keep z with ord_key(z) >= kmin
  const int64_t k = a.top_k ? a.top_k[row] : 0;
  if (k > 0 && k < V) {
    uint32_t prefix = 0, pmask = 0;
    int64_t remaining = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int b = tid; b < 256; b += nt) sh.hist.cnt[b] = 0;
      __syncthreads();
      for (int64_t i = tid; i < V; i += nt) {
        const uint32_t key = ord_key(lg[i] / t);
        if ((key & pmask) == prefix) atomicAdd(&sh.hist.cnt[(key >> shift) & 255], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        int64_t above = 0;
        int d = 255;
        for (; d > 0; --d) {
          if (above + (int64_t)sh.hist.cnt[d] >= remaining) break;
          above += sh.hist.cnt[d];
        }
        sh.bcast_u[0] = (uint32_t)d;
        sh.bcast_u[1] = (uint32_t)(remaining - above);
      }
      __syncthreads();
      prefix |= sh.bcast_u[0] << shift;
      pmask |= 255u << shift;
      remaining = sh.bcast_u[1];
      __syncthreads();
    }
    kmin = prefix;
  }

  // ---- top-p: smallest key whose mass at or below it exceeds 1 - p ----------------------------
  const float p = a.top_p ? a.top_p[row] : 1.0f;
  uint32_t cut = kmin;
  if (p < 1.0f) {
    float zl = 0.f;
    for (int64_t i = tid; i < V; i += nt) {
      const float z = lg[i] / t;
      if (ord_key(z) >= kmin) zl += expf(z - m);
    }
    const float zk = block_sum(zl, sh);
    const double wscale = kMassScale / (double)zk;
    const double tgt = (1.0 - (double)p) * kMassScale;
    const unsigned long long target = tgt <= 0.0 ? 0ull : (unsigned long long)tgt;
    uint32_t prefix = 0, pmask = 0;
    unsigned long long below = 0;
    bool found = true;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int b = tid; b < 256; b += nt) sh.hist.mass[b] = 0ull;
      __syncthreads();
      for (int64_t i = tid; i < V; i += nt) {
        const float z = lg[i] / t;
        const uint32_t key = ord_key(z);
        if (key >= kmin && (key & pmask) == prefix) {
          const unsigned long long w = (unsigned long long)((double)expf(z - m) * wscale);
          atomicAdd(&sh.hist.mass[(key >> shift) & 255], w);
        }
      }
      __syncthreads();
      if (tid == 0) {
        unsigned long long cum = below;
        int d = 0;
        bool hit = false;
        for (; d < 256; ++d) {
          if (cum + sh.hist.mass[d] > target) {
            hit = true;
            break;
          }
          cum += sh.hist.mass[d];
        }
        sh.bcast_u[0] = hit ? (uint32_t)d : 256u;
        sh.bcast_ull = cum;
      }
      __syncthreads();
      if (sh.bcast_u[0] == 256u) {  // rounding left no crossing: keep only the largest value
        found = false;
        break;
      }
      prefix |= sh.bcast_u[0] << shift;
      pmask |= 255u << shift;
      below = sh.bcast_ull;
      __syncthreads();
    }
    cut = found ? max(prefix, kmin) : ord_key(m);
  }

  // ---- output over the kept set {ord_key(z) >= cut} -------------------------------------------
  if (a.mode == SAMP_MASK) {
    float* o = a.out + row * a.ldo;
    for (int64_t i = tid; i < V; i += nt) {
      const float z = lg[i] / t;
      o[i] = ord_key(z) >= cut ? z : -INFINITY;
    }
    return;
  }
  float zl = 0.f;
  for (int64_t i = tid; i < V; i += nt) {
    const float z = lg[i] / t;
    if (ord_key(z) >= cut) zl += expf(z - m);
  }
  const float zsum = block_sum(zl, sh);
  if (a.mode == SAMP_PROBS) {
    float* o = a.out + row * a.ldo;
    for (int64_t i = tid; i < V; i += nt) {
      const float z = lg[i] / t;
      o[i] = ord_key(z) >= cut ? expf(z - m) / zsum : 0.f;
    }
    return;
  }
  const float* nz = a.noise + row * a.ldn;
  float bv = -1.f;
  int bi = 0x7fffffff;
  for (int64_t i = tid; i < V; i += nt) {
    const float z = lg[i] / t;
    if (ord_key(z) < cut) continue;
    const float s = (expf(z - m) / zsum) / fmaxf(nz[i], 1.17549435e-38f);  // noise clamped as the reference does
    if (s > bv) {
      bv = s;
      bi = (int)i;
    }
  }
  const int id = block_argmax(bv, bi, sh);
  if (tid == 0) a.ids[row] = id;
}

__global__ __launch_bounds__(kSampThreads) void sample_rows_kernel(SampArgs a) {
  __shared__ SampShared sh;
  sample_row(a, blockIdx.x, sh);
}

// ---- SAMPLE over vocabulary chunks -------------------------------------------------------------
// Rows with 0 < top_k <= kTopKFast (and greedy rows) are spread over chunk workgroups, so the
// whole GPU reads the logits once:
//  1. sample_chunk_kernel, one workgroup per (row, chunk of kCandChunk logits held in registers):
//     a greedy row's first argmax of the raw logits; a top-k row's candidates -- every logit at
//     or above the k-th largest of the 256 per-thread maxima (a lower bound on the chunk's k-th
//     largest; z = l / t keeps that order) and the few just below it whose z ties -- as (key,
//     index) pairs. The global k-th largest is at least every
//     chunk's k-th largest, so the union of the chunks' candidates holds every kept token, ties
//     included.
//  2. sample_finish_kernel, one workgroup per row: the greedy id from the chunks' argmaxes; else
//     the row's k-th largest among the candidates (radix select in LDS: 12, 12 and 8-bit
//     digits), the top-p cut over the kept set sorted
//     ascending (masses in 2^-44 fixed point, exact 64-bit sums, as the whole-row path), and the
//     exponential race over the final set -- noise read at the kept indices only. A row whose
//     chunks held more than kCandCap candidates each (long runs of equal values), or whose top-k
//     is outside (0, kTopKFast], takes the whole-row path instead.
constexpr int kCandThreads = 256;
constexpr int kCandPerThread = 40;
constexpr int kCandChunk = kCandThreads * kCandPerThread;  // logits per chunk workgroup
constexpr int kTopKFast = 256;
constexpr int kCandCap = 512;       // candidates kept per chunk
constexpr int kFinishCap = 8192;    // candidates the finishing workgroup takes per row (LDS)
constexpr int kMaxChunks = 64;      // chunks per row the finishing workgroup gathers (vocab <= 655,360)
constexpr int kFinishThreads = 256;  // (a row that falls back runs the whole-row path on these too)
static_assert(kCandThreads == 256 && kFinishThreads == 256, "the bounds take the k-th largest of 256 thread maxima");
static_assert(kMaxChunks == 64, "the finishing workgroup reads one chunk count per lane of a wavefront");
static_assert(kCandPerThread < 64, "a thread's candidate count fits six bits");

struct CandArgs {
  SampArgs a;
  int chunks;          // chunk workgroups per row
  uint32_t* cand_key;  // [rows][chunks][kCandCap]
  int32_t* cand_idx;   // [rows][chunks][kCandCap]
  int32_t* cand_cnt;   // [rows][chunks]: candidates, or -1 (row not chunked) / -2 (over kCandCap)
  float* arg_val;      // [rows][chunks]: greedy rows' chunk maximum
  int32_t* arg_idx;    // [rows][chunks]: and its first index (0x7fffffff: none)
};

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// The row's parameters for the chunked kernels, each read unconditionally (a missing array reads a
// constant default: temperature 1, top-k 0, top-p 1), so the loads issue together rather than one
// after another behind branches.
__constant__ float kDefaultOne = 1.0f;
__constant__ int32_t kDefaultTopK = 0;
__device__ __forceinline__ float row_temperature(const SampArgs& a, int64_t row) {
  return *(a.temperature ? a.temperature + row : &kDefaultOne);
}
__device__ __forceinline__ float row_top_p(const SampArgs& a, int64_t row) {
  return *(a.top_p ? a.top_p + row : &kDefaultOne);
}
__device__ __forceinline__ bool take_rows_chunked(const SampArgs& a, int64_t row, int64_t* k_out) {
  const int64_t k = *(a.top_k ? a.top_k + row : &kDefaultTopK);
  *k_out = k;
  return k > 0 && k <= kTopKFast && k < a.vocab;
}

// Inclusive suffix sum over the lanes of a wavefront: lane l gets the sum over lanes >= l.
__device__ __forceinline__ uint32_t wave_suffix_sum(uint32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_down((int)v, off);
    v += lane + off < 64 ? o : 0u;
  }
  return v;
}

// Inclusive suffix sums of v over the NT threads: thread t gets the sum over threads >= t. One
// barrier: per-wavefront scans, the wavefront totals through LDS (s_wave: NT / 64 entries).
template <int NT>
__device__ __forceinline__ uint32_t block_suffix_sum(uint32_t v, uint32_t* s_wave, uint32_t* total = nullptr) {
  const int w = threadIdx.x >> 6;
  const uint32_t in_wave = wave_suffix_sum(v);
  if ((threadIdx.x & 63) == 0) s_wave[w] = in_wave;
  __syncthreads();
  uint32_t later = 0, all = 0;
#pragma unroll
  for (int u = 0; u < NT / 64; ++u) {
    const uint32_t x = s_wave[u];
    later += u > w ? x : 0u;
    all += x;
  }
  if (total) *total = all;
  __syncthreads();
  return in_wave + later;
}

// Exclusive prefix sum of v over the threads of the workgroup (thread t gets the sum over threads
// < t): shuffles within each wavefront, the wavefront totals through LDS (s_w: one per wavefront).
__device__ __forceinline__ unsigned long long block_exclusive_scan_u64(unsigned long long v, unsigned long long* s_w) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  unsigned long long incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const unsigned long long o = __shfl_up(incl, off);
    incl += lane >= off ? o : 0ull;
  }
  if (lane == 63) s_w[w] = incl;
  __syncthreads();
  unsigned long long before = 0;
  for (int u = 0; u < w; ++u) before += s_w[u];
  (void)nw;
  __syncthreads();
  return before + incl - v;
}

// Histogram slot of bin b: one pad word per 64 bins (4096-bin digits) or per 4 bins (256-bin
// digits), so the wavefront scanning lane l's contiguous bins reads 64 different banks.
template <int NB>
__device__ __forceinline__ int hslot(uint32_t b) {
  return NB == 4096 ? (int)(b + (b >> 6)) : (int)(b + (b >> 2));
}
constexpr int kHistWords = 4096 + 64;  // slots of one level (the 256-bin level uses 320)

// The digit of the remaining-th largest key among the histogram's NB bins (bin index = digit):
// the largest d with count(digit >= d) >= remaining. Wavefront 0 alone scans (NB / 64
// contiguous bins per lane) and writes (d, remaining - count(digit > d)) to out[0..1]; one barrier.
template <int NB>
__device__ __forceinline__ void select_digit(const uint32_t* hist, uint32_t remaining, uint32_t* out) {
  constexpr int B = NB / 64;
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    uint32_t h[B];  // lane l's bins, read once (the scan below stays in registers)
    uint32_t tot = 0;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      h[b] = hist[hslot<NB>(l * B + b)];
      tot += h[b];
    }
    const uint32_t incl = wave_suffix_sum(tot);  // bins of lanes >= l
    const uint32_t above0 = incl - tot;          // bins of lanes > l
    if (above0 < remaining && incl >= remaining) {
      uint32_t above = above0, d = 0, rem = 0;
      bool hit = false;
#pragma unroll
      for (int b = B - 1; b >= 0; --b) {
        if (!hit && above + h[b] >= remaining) {
          hit = true;
          d = (uint32_t)(l * B + b);
          rem = remaining - above;
        }
        above += hit ? 0u : h[b];
      }
      out[0] = d;
      out[1] = rem;
    }
  }
  __syncthreads();
}

// Radix digits of the k-th largest key: 12, 12 and 8 bits, each with its own histogram region
// (hist: 3 x 4096 entries, cleared beforehand).
constexpr int kRadixShift[3] = {20, 8, 0};
constexpr uint32_t kRadixMask[3] = {4095u, 4095u, 255u};

// The kk-th largest of the n keys key_of(i) (1 <= kk <= n). NT threads, each visiting keys
// i = tid, tid + NT, ...; hist: 3 x kHistWords words.
template <int NT, typename KeyOf>
__device__ uint32_t radix_kth(KeyOf key_of, int n, uint32_t kk, uint32_t* hist, uint32_t* s_sel) {
  const int t = threadIdx.x;
  for (int b = t; b < 3 * kHistWords; b += NT) hist[b] = 0;
  __syncthreads();
  uint32_t prefix = 0, pmask = 0, remaining = kk;
#pragma unroll
  for (int lv = 0; lv < 3; ++lv) {
    uint32_t* h = hist + lv * kHistWords;
    for (int i = t; i < n; i += NT) {
      const uint32_t key = key_of(i);
      if ((key & pmask) == prefix) {
        const uint32_t d = (key >> kRadixShift[lv]) & kRadixMask[lv];
        atomicAdd(&h[lv < 2 ? hslot<4096>(d) : hslot<256>(d)], 1u);
      }
    }
    __syncthreads();
    if (lv < 2) select_digit<4096>(h, remaining, s_sel);
    else select_digit<256>(h, remaining, s_sel);
    prefix |= s_sel[0] << kRadixShift[lv];
    pmask |= kRadixMask[lv] << kRadixShift[lv];
    remaining = s_sel[1];
  }
  return prefix;
}

// A lower bound on the kk-th largest of 256 keys held four per lane by one wavefront (kk >= 1; 0
// when fewer than kk keys are nonzero): the largest r whose low 16 bits are zero with at least kk
// keys >= r, built from the top bit down, each trial counted with ballots (no LDS traffic, no
// barriers). It lies within the kk-th largest key's top 16 bits (sign, exponent and 7 mantissa
// bits: 2^-7 relative), so a bound taken on it admits only the few entries in that sliver, at
// half the dependent steps of the exact value.
__device__ __forceinline__ uint32_t wave_kth_of_256(uint4 v, uint32_t kk) {
  kk = __builtin_amdgcn_readfirstlane(kk);
  uint32_t r = 0;
#pragma unroll
  for (int bit = 31; bit >= 16; --bit) {
    const uint32_t tr = r | (1u << bit);
    const uint32_t cnt = (uint32_t)(__popcll(__ballot(v.x >= tr)) + __popcll(__ballot(v.y >= tr)) +
                                    __popcll(__ballot(v.z >= tr)) + __popcll(__ballot(v.w >= tr)));
    r = __builtin_amdgcn_readfirstlane(cnt >= kk ? tr : r);
  }
  return r;
}

// Workgroup reductions of the chunked kernels (256 threads, four wavefronts) on DPP and gfx950's
// row swaps within each wavefront -- VALU only, no LDS round trip per step as with ds_bpermute
// shuffles -- and one LDS exchange of the four wavefront results.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(r[0], r[1]);
  r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(r[0], r[1]);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dpp_u32<0xB1>(v));
  v = min(v, dpp_u32<0x4E>(v));
  v = min(v, dpp_u32<0x141>(v));
  v = min(v, dpp_u32<0x140>(v));
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = min(r[0], r[1]);
  r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return min(r[0], r[1]);
}
// The first index of the largest value within a wavefront: (v, i) pairs, i >= 0.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  const float m = wave_max(v);
  i = (int)wave_min_u32(v == m ? (uint32_t)i : 0x7fffffffu);
  v = m;
}
// Sum over the workgroup in a fixed order (s_red: four floats, not reused before a later barrier).
__device__ __forceinline__ float wg_sum(float v, float* s_red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
}
// The first index of the largest value over the workgroup (s_v, s_i: four entries each).
__device__ __forceinline__ int wg_argmax(float v, int i, float* s_v, int* s_i) {
  wave_argmax(v, i);
  if ((threadIdx.x & 63) == 0) {
    s_v[threadIdx.x >> 6] = v;
    s_i[threadIdx.x >> 6] = i;
  }
  __syncthreads();
  float bv = s_v[0];
  int bi = s_i[0];
#pragma unroll
  for (int w = 1; w < 4; ++w)
    if (s_v[w] > bv || (s_v[w] == bv && s_i[w] < bi)) {
      bv = s_v[w];
      bi = s_i[w];
    }
  return bi;
}
// Exclusive prefix sum over the workgroup's threads of small counts v < 2^NB, and the total:
// bit-sliced ballots counted below each lane (mbcnt), the wavefront totals through LDS (s_wave:
// four entries, not reused before a later barrier).
template <int NB>
__device__ __forceinline__ uint32_t wg_prefix_small(uint32_t v, uint32_t* s_wave, uint32_t* all) {
  uint32_t ex = 0, tot = 0;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const unsigned long long m = __ballot((v >> b) & 1u);
    ex += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) << b;
    tot += (uint32_t)__popcll(m) << b;
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_wave[w] = tot;
  __syncthreads();
  uint32_t before = 0, a = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t x = s_wave[u];
    before += u < w ? x : 0u;
    a += x;
  }
  *all = a;
  return before + ex;
}

__global__ __launch_bounds__(kCandThreads) void sample_chunk_kernel(CandArgs c) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tmax[kCandThreads];
  __shared__ uint32_t s_scan[kCandThreads / 64];
  __shared__ uint32_t s_sel[2];
  __shared__ float fred[kCandThreads / 64];
  __shared__ int ired[kCandThreads / 64];
  __shared__ uint32_t s_ck[kCandThreads / 64][kCandCap];
  __shared__ int32_t s_ci[kCandThreads / 64][kCandCap];
  const SampArgs& a = c.a;
  const int64_t row = blockIdx.y;
  const int chunk = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)chunk * kCandChunk;
  const int n = (int)min((int64_t)kCandChunk, a.vocab - base);
  const float* lg = a.logits + row * a.ld + base;
  const int64_t slot = row * c.chunks + chunk;

  // The chunk's logits are loaded first, every load issued before anything waits (slots past the
  // row re-read its last entry): a load under a branch, or after one that needs the row's flags,
  // would wait for what was issued before it.
  float vals[kCandPerThread];
#pragma unroll
  for (int i = 0; i < kCandPerThread; ++i) vals[i] = __builtin_nontemporal_load(lg + min(i * kCandThreads + tid, n - 1));
  if (a.greedy && a.greedy[row]) {  // first index of the largest raw logit in the chunk
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) {  // ascending index: the first of equal maxima stays
      const int e = i * kCandThreads + tid;
      if (e < n && vals[i] > bv) {
        bv = vals[i];
        bi = (int)(base + e);
      }
    }
    wave_argmax(bv, bi);
    if ((tid & 63) == 0) { fred[tid >> 6] = bv; ired[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < kCandThreads / 64; ++w)
        if (fred[w] > bv || (fred[w] == bv && ired[w] < bi)) { bv = fred[w]; bi = ired[w]; }
      c.arg_val[slot] = bv;
      c.arg_idx[slot] = bi;
    }
    return;
  }
  int64_t k;
  if (!take_rows_chunked(a, row, &k)) {
    if (tid == 0) c.cand_cnt[slot] = -1;
    return;
  }
  const float t = row_temperature(a, row);
  // The bound is found on the raw logits l: z = l / t (t > 0) orders the entries as l does, up to
  // rounding ties, so no entry is divided here. Slots past the row hold NaN, which no comparison
  // keeps (the row's last chunk only).
  if (n < kCandChunk) {
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i)
      if (i * kCandThreads + tid >= n) vals[i] = __builtin_nanf("");
  }
  // A lower bound on the chunk's k-th largest logit: L <= the k-th largest of the 256 per-thread
  // maxima (k distinct entries are at or above it; a thread without entries holds -inf).
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < kCandPerThread; ++i) tmax = fmaxf(tmax, vals[i]);
  s_tmax[tid] = ord_key(tmax);
  __syncthreads();
  if (tid < 64) {  // bounding the k-th largest of the 256 maxima, bit by bit on wavefront 0
    const uint32_t b = wave_kth_of_256(((const uint4*)s_tmax)[tid], (uint32_t)k);
    if (tid == 0) s_sel[0] = b;
  }
  __syncthreads();
  const float lb = key_value(s_sel[0]);
  // Candidates: l >= L' = L - 2^-20 |L| - 2^-126, a superset of the chunk's top k that also holds
  // every entry whose z rounds up to L / t (entries below L' give z < L / t: the margin is far
  // wider than a rounding step of z). With L or L / t infinite, every entry is a candidate.
  const float lq = isfinite(lb) && isfinite(lb / t) ? lb - fabsf(lb) * 0x1p-20f - 0x1p-126f : -INFINITY;
  // Candidates staged per wavefront in LDS, in a deterministic order (slot, then lane): one
  // compare per slot gives the wavefront's mask, and only slots that hold candidates write.
  const int wv = tid >> 6;
  uint32_t wn = 0;  // the wavefront's candidates so far
#pragma unroll
  for (int i = 0; i < kCandPerThread; ++i) {
    const bool cand = vals[i] >= lq;
    const unsigned long long m = __ballot(cand);
    if (m != 0ull) {
      const uint32_t pos = wn + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      if (cand && pos < (uint32_t)kCandCap) {
        s_ck[wv][pos] = ord_key(vals[i]);  // the raw logit's key: the finishing kernel divides by t
        s_ci[wv][pos] = (int32_t)(base + i * kCandThreads + tid);
      }
      wn += (uint32_t)__popcll(m);
    }
  }
  if ((tid & 63) == 0) s_scan[wv] = wn;
  __syncthreads();
  const uint32_t o1 = s_scan[0], o2 = o1 + s_scan[1], o3 = o2 + s_scan[2], all = o3 + s_scan[3];
  if (all > (uint32_t)kCandCap) {
    if (tid == 0) c.cand_cnt[slot] = -2;
    return;
  }
  // The wavefronts' runs one after another, written out coalesced.
  uint32_t* ck = c.cand_key + slot * kCandCap;
  int32_t* ci = c.cand_idx + slot * kCandCap;
  for (uint32_t j = tid; j < all; j += kCandThreads) {
    const int src = j >= o3 ? 3 : j >= o2 ? 2 : j >= o1 ? 1 : 0;
    const uint32_t at = j - (src == 3 ? o3 : src == 2 ? o2 : src == 1 ? o1 : 0u);
    ck[j] = s_ck[src][at];
    ci[j] = s_ci[src][at];
  }
  if (tid == 0) c.cand_cnt[slot] = (int32_t)all;
}

// LDS of the finishing workgroup's fast path.
struct FinishShared {
  __attribute__((aligned(16))) uint32_t tmax[kFinishThreads];  // threads' maxima
  __attribute__((aligned(16))) uint32_t pk[kFinishThreads];    // P: z keys (zeros up to a multiple of 16)
  int32_t pi[kFinishThreads];                                  // P: indices
  __attribute__((aligned(16))) unsigned long long mass[kFinishThreads];
  uint32_t scan[4];
  uint32_t sel[2];
  float red0[4], red1[4], argv[4];
  int argi[4];
};

__device__ __forceinline__ uint32_t count_gt(uint4 o, uint32_t kv) {
  return (o.x > kv ? 1u : 0u) + (o.y > kv ? 1u : 0u) + (o.z > kv ? 1u : 0u) + (o.w > kv ? 1u : 0u);
}
__device__ __forceinline__ unsigned long long mass_le(uint4 o, ulonglong2 m01, ulonglong2 m23, uint32_t kv) {
  return (o.x <= kv ? m01.x : 0ull) + (o.y <= kv ? m01.y : 0ull) + (o.z <= kv ? m23.x : 0ull) +
         (o.w <= kv ? m23.y : 0ull);
}

// The finish of a row from P: np <= kFinishThreads candidates (z keys in fs.pk, indices in fs.pi,
// one per thread, fs.pk zero-padded to a multiple of 16) that hold every entry of the row's top-k
// set K, mkey = the largest z key. An entry is in K when fewer than k entries of P are greater.
// Top-p keeps x in K when the mass of K at or below x (every entry of equal value included)
// exceeds (1 - p) of K's mass: masses e = exp(z - m) in 2^-40 fixed point (exact, order-free
// integer sums), each thread summing over P for its own key -- nothing is sorted, and since that
// mass grows with x the kept entries are exactly those above the cut, found without a search (no
// entry qualifying by rounding: the largest alone). Then the exponential race over the kept set:
// the first index of the largest e / noise (the softmax normalisation is common to every entry).
// The loops read 16 entries per step (four 16-byte LDS reads in flight).
__device__ void finish_p(FinishShared& fs, int np, uint32_t k, float p, const float* nz, uint32_t mkey,
                         int64_t* id_out) {
  const int tid = threadIdx.x;
  const bool live = tid < np;
  const int np16 = (np + 15) & ~15;
  uint32_t kv = 0, gt = 0;
  int iv = 0;
  float nzv = 1.f;
  if (live) {
    kv = fs.pk[tid];
    iv = fs.pi[tid];
    nzv = nz[iv];  // issued before the count below, which hides its latency
    for (int j = 0; j < np16; j += 16) {
      const uint4 o0 = *(const uint4*)(fs.pk + j), o1 = *(const uint4*)(fs.pk + j + 4);
      const uint4 o2 = *(const uint4*)(fs.pk + j + 8), o3 = *(const uint4*)(fs.pk + j + 12);
      gt += count_gt(o0, kv) + count_gt(o1, kv) + count_gt(o2, kv) + count_gt(o3, kv);
    }
  }
  const bool in_k = live && gt < k;
  const float e = in_k ? expf(key_value(kv) - key_value(mkey)) : 0.f;
  bool fin = in_k;
  if (p < 1.0f) {
    fs.mass[tid] = in_k ? (unsigned long long)((double)e * 0x1p40) : 0ull;  // (padding: 0)
    __syncthreads();
    if (in_k) {  // (the padding keys 0 are <= kv; their masses are 0)
      unsigned long long cum = 0, tot = 0;
      for (int j = 0; j < np16; j += 16) {
        const uint4 o0 = *(const uint4*)(fs.pk + j), o1 = *(const uint4*)(fs.pk + j + 4);
        const uint4 o2 = *(const uint4*)(fs.pk + j + 8), o3 = *(const uint4*)(fs.pk + j + 12);
        const ulonglong2* mm = (const ulonglong2*)(fs.mass + j);
        cum += mass_le(o0, mm[0], mm[1], kv) + mass_le(o1, mm[2], mm[3], kv) + mass_le(o2, mm[4], mm[5], kv) +
               mass_le(o3, mm[6], mm[7], kv);
#pragma unroll
        for (int u = 0; u < 8; ++u) tot += mm[u].x + mm[u].y;
      }
      fin = (double)cum > (1.0 - (double)p) * (double)tot || kv == mkey;
    }
  }
  float bv = -1.f;
  int bi = 0x7fffffff;
  if (fin) {
    bv = e / fmaxf(nzv, 1.17549435e-38f);
    bi = iv;
  }
  const int id = wg_argmax(bv, bi, fs.argv, fs.argi);
  if (tid == 0) *id_out = id;
}

// A lower bound on the k-th largest of the 256 threads' maxima in fs.tmax and the largest of them,
// by wavefront 0, into fs.sel.
__device__ __forceinline__ void select_bound(FinishShared& fs, uint32_t k) {
  if (threadIdx.x < 64) {
    const uint4 v = ((const uint4*)fs.tmax)[threadIdx.x];
    const uint32_t b = wave_kth_of_256(v, k);
    const uint32_t mx = wave_max_u32(max(max(v.x, v.y), max(v.z, v.w)));
    if (threadIdx.x == 0) {
      fs.sel[0] = b;
      fs.sel[1] = mx;
    }
  }
  __syncthreads();
}

// The margin under a bound L on raw logits: entries below L' = L - 2^-20 |L| - 2^-126 give
// z = l / t below L / t (the margin is far wider than a rounding step of z), so they are not in
// the top-k of a row with k entries at or above L. With L or L / t not finite: -inf (every entry).
__device__ __forceinline__ float bound_margin(float lb, float t) {
  return isfinite(lb) && isfinite(lb / t) ? lb - fabsf(lb) * 0x1p-20f - 0x1p-126f : -INFINITY;
}

// The finish of a row of at most NS chunks whose candidate counts are all at most kFinishThreads,
// the candidates held in registers from one round of loads: wavefront w takes chunks w, w + 4, ...
// (lane l: candidates l, l + 64, l + 128, l + 192 of each), so every load reads 64 consecutive
// candidates and the row's few candidates per chunk spread over the four wavefronts. B = a bound on
// the k-th largest of the threads' maxima of raw-logit keys (k distinct candidates at or above it),
// P = the candidates at or above its margin (usually about k), divided by t and compacted into
// LDS, then finish_p. Returns false, every thread agreeing and nothing written, when a count or P
// does not fit.
template <int NS>
__device__ bool finish_regs(const CandArgs& c, int64_t row, uint32_t k, float t, float p, const float* nz,
                            FinishShared& fs) {
  constexpr int NT = kFinishThreads;
  constexpr int NC = NS / 4;  // chunks per wavefront
  static_assert(NS % 4 == 0 && NT == 256, "four wavefronts, four 64-candidate blocks per chunk");
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63;
  const int nch = c.chunks;
  int cn[NC];
  uint32_t rk[NS];
  int32_t ri[NS];
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {  // every load issued before any is used (chunks past the row re-read the last)
    const int64_t sl = row * nch + min(cc * 4 + w, nch - 1);
    cn[cc] = c.cand_cnt[sl];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      rk[cc * 4 + b] = c.cand_key[sl * kCandCap + l + 64 * b];
      ri[cc * 4 + b] = c.cand_idx[sl * kCandCap + l + 64 * b];
    }
  }
  uint32_t tm = 0;
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    const int n = cc * 4 + w < nch ? cn[cc] : 0;
    if (n < 0 || n > NT) tm = 0xffffffffu;  // a count that does not fit: flagged as the maximum
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int q = cc * 4 + b;
      if (l + 64 * b < n) rk[q] = ord_key(key_value(rk[q]) / t);  // z = logits / temperature (IEEE division)
      else rk[q] = 0u;  // no candidate (below every candidate's key)
      tm = max(tm, rk[q]);
    }
  }
  fs.tmax[tid] = tm;
  __syncthreads();
  select_bound(fs, k);
  const uint32_t mxk = fs.sel[1];
  if (mxk == 0xffffffffu) return false;  // uniform (candidates are never NaN: no key reaches it)
  const uint32_t bnd = fs.sel[0];
  uint32_t mine = 0;
#pragma unroll
  for (int q = 0; q < NS; ++q) mine += rk[q] != 0u && rk[q] >= bnd ? 1u : 0u;
  uint32_t np;
  uint32_t at = wg_prefix_small<6>(mine, fs.scan, &np);  // P entries of threads < tid
  if (np > (uint32_t)NT) return false;  // uniform
  if (tid >= (int)np && tid < (int)((np + 15) & ~15u)) fs.pk[tid] = 0u;  // padding for 16-wide reads
#pragma unroll
  for (int q = 0; q < NS; ++q)
    if (rk[q] != 0u && rk[q] >= bnd) {
      fs.pk[at] = rk[q];
      fs.pi[at] = ri[q];
      ++at;
    }
  __syncthreads();
  finish_p(fs, (int)np, k, p, nz, mxk, &c.a.ids[row]);
  return true;
}

// P from the nc candidates gathered into LDS (z keys): B = a bound on the k-th largest of the
// threads' maxima over candidates tid, tid + NT, ...; P = the candidates at or above B, compacted
// into fs. Returns np, or -1 (every thread agreeing) when P does not fit one per thread.
__device__ int p_from_lds(const uint32_t* s_key, const int32_t* s_idx, int nc, uint32_t k, FinishShared& fs,
                          uint32_t* mkey) {
  constexpr int NT = kFinishThreads;
  const int tid = threadIdx.x;
  uint32_t tm = 0;
  for (int i = tid; i < nc; i += NT) tm = max(tm, s_key[i]);
  fs.tmax[tid] = tm;
  __syncthreads();
  select_bound(fs, k);
  const uint32_t bnd = fs.sel[0];
  *mkey = fs.sel[1];
  uint32_t mine = 0;
  for (int i = tid; i < nc; i += NT) mine += s_key[i] >= bnd ? 1u : 0u;
  uint32_t np;
  uint32_t w = wg_prefix_small<6>(mine, fs.scan, &np);
  if (np > (uint32_t)NT) return -1;
  if (tid >= (int)np && tid < (int)((np + 15) & ~15u)) fs.pk[tid] = 0u;  // padding for 16-wide reads
  for (int i = tid; i < nc; i += NT)
    if (s_key[i] >= bnd) {
      fs.pk[w] = s_key[i];
      fs.pi[w] = s_idx[i];
      ++w;
    }
  __syncthreads();
  return (int)np;
}

__global__ __launch_bounds__(kFinishThreads) void sample_finish_kernel(CandArgs c) {
  __shared__ SampShared sh;
  __shared__ uint32_t s_key[kFinishCap];
  __shared__ int32_t s_idx[kFinishCap];
  __shared__ __attribute__((aligned(16))) uint32_t hist[3 * kHistWords];
  __shared__ uint32_t s_scan[kFinishThreads / 64];
  __shared__ uint32_t s_sel[2];
  __shared__ int s_info[2];
  __shared__ int s_off[kMaxChunks];
  __shared__ uint32_t s_sort[kFinishCap];
  __shared__ __attribute__((aligned(16))) unsigned long long s_mass[kFinishThreads];
  __shared__ FinishShared fs;
  const SampArgs& a = c.a;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t slot0 = row * c.chunks;

  if (a.greedy && a.greedy[row]) {  // the first index of the largest chunk maximum
    if (tid < 64) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int ch = tid; ch < c.chunks; ch += 64) {  // ascending chunks: equal maxima keep the first
        const float v = c.arg_val[slot0 + ch];
        const int i = c.arg_idx[slot0 + ch];
        if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
      }
      wave_argmax(bv, bi);
      if (tid == 0) a.ids[row] = bi == 0x7fffffff ? 0 : bi;  // a row of -inf: index 0, as argmax
    }
    return;
  }
  int64_t k;
  take_rows_chunked(a, row, &k);  // (a row that was not chunked has a negative count below)
  const float t = row_temperature(a, row);
  const float p = row_top_p(a, row);
  const float* nz = a.noise + row * a.ldn;
  if (c.chunks <= 16) {
    if (finish_regs<16>(c, row, (uint32_t)k, t, p, nz, fs)) return;
  } else if (c.chunks <= 32) {
    if (finish_regs<32>(c, row, (uint32_t)k, t, p, nz, fs)) return;
  }
  // Every candidate into LDS. Lane l of the first wavefront reads chunk l's count; the offsets are
  // an exclusive scan over the lanes. A row that was not chunked, or overflowed somewhere, takes
  // the whole-row path.
  if (tid < 64) {
    int cnt = tid < c.chunks ? c.cand_cnt[slot0 + tid] : 0;
    const bool bad = __any(cnt < 0);
    cnt = max(cnt, 0);
    const uint32_t suffix = wave_suffix_sum((uint32_t)cnt);  // chunks >= tid
    const uint32_t total = (uint32_t)__shfl((int)suffix, 0);
    s_off[tid] = (int)(total - suffix);
    if (tid == 0) {
      s_info[0] = !bad && c.chunks <= kMaxChunks && total <= (uint32_t)kFinishCap;
      s_info[1] = (int)total;
    }
  }
  __syncthreads();
  if (!s_info[0]) {
    sample_row(a, row, sh);
    return;
  }
  const int nc = s_info[1];
  // Gather the candidates (chunk order, then their order within the chunk): candidate j of the
  // row comes from the chunk whose offset range holds it (a binary search over the offsets).
  // The loads of a thread's candidates are issued unconditionally (a load under a branch is
  // waited for before the next one).
  {
    const int nch = min(c.chunks, kMaxChunks);
#pragma unroll 4
    for (int j0 = 0; j0 < kFinishCap; j0 += kFinishThreads) {
      if (j0 >= nc) break;  // uniform
      const int j = min(j0 + tid, nc - 1);
      int lo = 0, hi = nch - 1;  // the last chunk whose offset is <= j
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_off[mid] <= j) lo = mid;
        else hi = mid - 1;
      }
      const int64_t src = (slot0 + lo) * kCandCap + (j - s_off[lo]);
      const uint32_t kv = c.cand_key[src];
      const int32_t iv = c.cand_idx[src];
      if (j0 + tid < nc) {
        s_key[j] = ord_key(key_value(kv) / t);  // z = logits / temperature (IEEE division)
        s_idx[j] = iv;
      }
    }
  }
  __syncthreads();
  {
    uint32_t mkey;
    const int np = p_from_lds(s_key, s_idx, nc, (uint32_t)k, fs, &mkey);
    if (np >= 0) {
      finish_p(fs, np, (uint32_t)k, p, nz, mkey, &a.ids[row]);
      return;
    }
  }
  // Many candidates at the bound (ties): the k-th largest by radix select over all of them.
  const uint32_t kth = radix_kth<kFinishThreads>([&](int i) { return s_key[i]; }, nc, (uint32_t)k, hist, s_sel);
  // The kept set K = {key >= kth}; its largest value m.
  uint32_t kmax = 0;
  for (int i = tid; i < nc; i += kFinishThreads) kmax = max(kmax, s_key[i]);
  const float m = block_max(key_value(kmax == 0 ? ord_key(-INFINITY) : kmax), sh);
  // ---- top-p over K: ascending sort of K's keys, masses, the cut ----
  uint32_t cut = kth;
  if (p < 1.0f) {
    // Compact K to the front in candidate order (thread t takes a contiguous range of R).
    const int R = (nc + kFinishThreads - 1) / kFinishThreads;
    uint32_t mine = 0;
    for (int i = tid * R; i < min(nc, tid * R + R); ++i) mine += s_key[i] >= kth ? 1u : 0u;
    const uint32_t incl = block_suffix_sum<kFinishThreads>(mine, s_scan);
    if (tid == 0) s_info[1] = (int)incl;
    __syncthreads();
    const int nk = s_info[1];
    {
      int w = nk - (int)incl;  // kept candidates of threads < tid
      for (int i = tid * R; i < min(nc, tid * R + R); ++i)
        if (s_key[i] >= kth) s_sort[w++] = s_key[i];
    }
    __syncthreads();
    // Sort K ascending: by rank (one pass of broadcast reads per entry, no barriers) up to one
    // entry per thread, else bitonic (padded with keys that sort last).
    if (nk <= kFinishThreads) {
      uint32_t kv = 0, rank = 0;
      if (tid < nk) {
        kv = s_sort[tid];
        for (int j = 0; j < nk; ++j) {
          const uint32_t o = s_sort[j];
          rank += (o < kv) || (o == kv && j < tid);
        }
      }
      __syncthreads();
      if (tid < nk) s_sort[rank] = kv;
      __syncthreads();
    } else {
      int np2 = 1;
      while (np2 < nk) np2 <<= 1;
      for (int i = nk + tid; i < np2; i += kFinishThreads) s_sort[i] = 0xffffffffu;
      __syncthreads();
      for (int size = 2; size <= np2; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          for (int i = tid; i < np2; i += kFinishThreads) {
            const int jx = i ^ stride;
            if (jx > i) {
              const bool up = (i & size) == 0;
              const uint32_t x = s_sort[i], y = s_sort[jx];
              if ((x > y) == up) { s_sort[i] = y; s_sort[jx] = x; }
            }
          }
          __syncthreads();
        }
    }
    // Z_K in a fixed order (strided per thread over the sorted keys, then a fixed tree)
    float zl = 0.f;
    for (int i = tid; i < nk; i += kFinishThreads) zl += expf(key_value(s_sort[i]) - m);
    const float zk = block_sum(zl, sh);
    const double wscale = kMassScale / (double)zk;
    const double tgt = (1.0 - (double)p) * kMassScale;
    const unsigned long long target = tgt <= 0.0 ? 0ull : (unsigned long long)tgt;
    // Masses in 2^-44 fixed point and their prefix sums over the sorted keys (exact, order-free
    // 64-bit integers): thread t sums its contiguous range, an exclusive scan over the threads.
    const int R2 = (nk + kFinishThreads - 1) / kFinishThreads;
    unsigned long long loc = 0;
    for (int i = tid * R2; i < min(nk, tid * R2 + R2); ++i)
      loc += (unsigned long long)((double)expf(key_value(s_sort[i]) - m) * wscale);
    unsigned long long cum = block_exclusive_scan_u64(loc, s_mass);
    // The cut: the smallest key whose mass at or below it (every entry of equal value included)
    // exceeds the target -- the first value group whose inclusive sum at its last entry does.
    uint32_t best = 0xffffffffu;
    for (int i = tid * R2; i < min(nk, tid * R2 + R2); ++i) {
      cum += (unsigned long long)((double)expf(key_value(s_sort[i]) - m) * wscale);
      const bool group_end = i + 1 >= nk || s_sort[i + 1] != s_sort[i];
      if (group_end && cum > target) {
        best = s_sort[i];
        break;
      }
    }
    if (tid == 0) s_sel[0] = 0xffffffffu;
    __syncthreads();
    if (best != 0xffffffffu) atomicMin(&s_sel[0], best);
    __syncthreads();
    const uint32_t found = s_sel[0];
    cut = found == 0xffffffffu ? ord_key(m) : max(found, kth);  // no crossing (rounding): the largest only
    __syncthreads();
  }
  // ---- the exponential race over the final set ----
  float zl = 0.f;
  for (int i = tid; i < nc; i += kFinishThreads)
    if (s_key[i] >= cut) zl += expf(key_value(s_key[i]) - m);
  const float zsum = block_sum(zl, sh);
  float bv = -1.f;
  int bi = 0x7fffffff;
  for (int i = tid; i < nc; i += kFinishThreads) {
    if (s_key[i] < cut) continue;
    const int idx = s_idx[i];
    const float sc = (expf(key_value(s_key[i]) - m) / zsum) / fmaxf(nz[idx], 1.17549435e-38f);
    if (sc > bv || (sc == bv && idx < bi)) {
      bv = sc;
      bi = idx;
    }
  }
  const int id = block_argmax(bv, bi, sh);
  if (tid == 0) a.ids[row] = id;
}

// ---- speculative-decoding verification (spec/rejection.py) ------------------------------------

// Greedy verification from the target's own picks (spec/rejection.py:27-40): accepted = length of
// the leading run of drafts equal to the target's argmax at their position (among the real ones),
// next = the target's pick right after the run (a correction, or the bonus token).
__global__ void verify_greedy_kernel(const int64_t* __restrict__ target_ids, int k, const int64_t* __restrict__ drafts,
                                     const int64_t* __restrict__ num_drafts, int b, int64_t* __restrict__ accepted,
                                     int64_t* __restrict__ next_token) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= b) return;
  const int64_t* tgt = target_ids + (int64_t)i * (k + 1);
  const int64_t* dr = drafts + (int64_t)i * k;
  const int64_t n = num_drafts[i];
  int a = 0;
  while (a < k && a < n && tgt[a] == dr[a]) ++a;
  accepted[i] = a;
  next_token[i] = tgt[a];
}

// Rejection sampling (spec/rejection.py:43-79), one workgroup per sequence. p_i(d_i) / q_i(d_i)
// (q = 1 for a deterministic proposer) against uniform[i], the leading accepted run a, then a
// token from normalize(max(0, p_a - q_a)) (p_a with the rejected draft zeroed when q is one-hot)
// after a rejection, or from p_a itself when every real draft was accepted (the bonus token);
// normalize falls back to p_a when the residual is empty. The token is the first argmax of
// dist / noise.
__global__ __launch_bounds__(kSampThreads) void verify_sampled_kernel(
    const float* __restrict__ target_probs, int k, int64_t vocab, const int64_t* __restrict__ drafts,
    const int64_t* __restrict__ num_drafts, const float* __restrict__ draft_probs, const float* __restrict__ uniform,
    const float* __restrict__ noise, int64_t* __restrict__ accepted, int64_t* __restrict__ next_token) {
  __shared__ SampShared sh;
  __shared__ int s_acc;
  const int64_t b = blockIdx.x;
  const float* tp = target_probs + b * (int64_t)(k + 1) * vocab;
  const float* dp = draft_probs ? draft_probs + b * (int64_t)k * vocab : nullptr;
  const int64_t* dr = drafts + b * k;
  if (threadIdx.x == 0) {
    const int64_t n = num_drafts[b];
    int a = 0;
    while (a < k) {
      int64_t d = dr[a];
      d = d < 0 ? 0 : (d >= vocab ? vocab - 1 : d);  // memory safety only: draft ids are vocabulary ids
      const float pd = tp[(int64_t)a * vocab + d];
      const float ratio = dp ? pd / fmaxf(dp[(int64_t)a * vocab + d], 1e-20f) : pd;
      if (!(a < n && uniform[b * k + a] < fminf(ratio, 1.0f))) break;
      ++a;
    }
    s_acc = a;
  }
  __syncthreads();
  const int a = s_acc;
  const bool rejected = a < num_drafts[b];
  const int at = min(a, k - 1);
  const float* prow = tp + (int64_t)a * vocab;
  const float* qrow = dp ? dp + (int64_t)at * vocab : nullptr;
  const int64_t drop = k > 0 ? dr[at] : -1;
  auto dist = [&](int64_t i) -> float {
    const float pv = prow[i];
    if (!rejected) return pv;
    if (qrow) return fmaxf(pv - qrow[i], 0.f);
    return i == drop ? 0.f : pv;
  };
  float tl = 0.f;
  for (int64_t i = threadIdx.x; i < vocab; i += kSampThreads) tl += dist(i);
  const float total = block_sum(tl, sh);
  const float* nz = noise + b * vocab;
  float bv = -1.f;
  int bi = 0x7fffffff;
  for (int64_t i = threadIdx.x; i < vocab; i += kSampThreads) {
    const float dv = total > 0.f ? dist(i) / fmaxf(total, 1e-20f) : prow[i];
    const float sc = dv / fmaxf(nz[i], 1.17549435e-38f);
    if (sc > bv) {
      bv = sc;
      bi = (int)i;
    }
  }
  const int id = block_argmax(bv, bi, sh);
  if (threadIdx.x == 0) {
    accepted[b] = a;
    next_token[b] = id;
  }
}

static int sample_launch(SampArgs& a, int64_t rows, hipStream_t s, const char* what) {
  if (rows == 0) return MSA_OK;
  if (rows < 0 || rows > 0x7fffffff || a.vocab <= 0 || a.vocab > 0x7fffffff || !a.logits || a.ld < a.vocab)
    return fail(MSA_ERR_INVALID, std::string(what) + ": bad shape or null logits");
  hipLaunchKernelGGL(sample_rows_kernel, dim3((unsigned)rows), dim3(kSampThreads), 0, s, a);
  return check_launch(what);
}

static int64_t sample_chunks(int64_t vocab) { return (vocab + kCandChunk - 1) / kCandChunk; }

// Workspace of the chunked SAMPLE path: per (row, chunk) kCandCap (key, index) pairs, the count,
// the greedy maximum and its index.
static size_t sample_ws_bytes(int64_t rows, int64_t vocab) {
  const size_t slots = (size_t)rows * (size_t)sample_chunks(vocab);
  return slots * kCandCap * 2 * sizeof(uint32_t) + slots * 3 * sizeof(uint32_t);
}

}  // namespace msa

using namespace msa;

extern "C" int msa_top_k_top_p_mask(const float* logits, int64_t ld, int64_t rows, int64_t vocab,
                                    const int32_t* top_k, const float* top_p, float* out, int64_t ldo,
                                    msa_stream_t stream) {
  if (!out || ldo < vocab) return fail(MSA_ERR_INVALID, "msa_top_k_top_p_mask: bad out");
  SampArgs a{};
  a.logits = logits; a.ld = ld; a.vocab = vocab; a.top_k = top_k; a.top_p = top_p; a.out = out; a.ldo = ldo;
  a.mode = SAMP_MASK;
  return sample_launch(a, rows, (hipStream_t)stream, "msa_top_k_top_p_mask");
}

extern "C" int msa_sampling_probs(const float* logits, int64_t ld, int64_t rows, int64_t vocab, const float* temperature,
                                  const int32_t* top_k, const float* top_p, float* probs, int64_t ldp,
                                  msa_stream_t stream) {
  if (!probs || ldp < vocab) return fail(MSA_ERR_INVALID, "msa_sampling_probs: bad probs");
  SampArgs a{};
  a.logits = logits; a.ld = ld; a.vocab = vocab; a.temperature = temperature; a.top_k = top_k; a.top_p = top_p;
  a.out = probs; a.ldo = ldp; a.mode = SAMP_PROBS;
  return sample_launch(a, rows, (hipStream_t)stream, "msa_sampling_probs");
}

extern "C" size_t msa_sample_workspace_size(int64_t rows, int64_t vocab) {
  if (rows <= 0 || rows > 65535 || vocab <= 0 || vocab > 0x7fffffff) return 0;
  return sample_ws_bytes(rows, vocab);
}

extern "C" int msa_sample(const float* logits, int64_t ld, int64_t rows, int64_t vocab, const float* temperature,
                          const int32_t* top_k, const float* top_p, const uint8_t* greedy, const float* noise,
                          int64_t ldn, int64_t* out_ids, void* workspace, size_t workspace_bytes, msa_stream_t stream) {
  if (!out_ids || !noise || ldn < vocab) return fail(MSA_ERR_INVALID, "msa_sample: bad noise / out_ids");
  SampArgs a{};
  a.logits = logits; a.ld = ld; a.vocab = vocab; a.temperature = temperature; a.top_k = top_k; a.top_p = top_p;
  a.greedy = greedy; a.noise = noise; a.ldn = ldn; a.ids = out_ids; a.mode = SAMP_SAMPLE;
  if (workspace == nullptr || rows == 0) return sample_launch(a, rows, (hipStream_t)stream, "msa_sample");
  if (rows < 0 || rows > 65535 || vocab <= 0 || vocab > 0x7fffffff || !logits || ld < vocab)
    return fail(MSA_ERR_INVALID, "msa_sample: bad shape or null logits (the chunked path takes rows <= 65535)");
  if (workspace_bytes < sample_ws_bytes(rows, vocab))
    return fail(MSA_ERR_WORKSPACE, "msa_sample: workspace smaller than msa_sample_workspace_size");
  CandArgs c{};
  c.a = a;
  c.chunks = (int)sample_chunks(vocab);
  const size_t slots = (size_t)rows * c.chunks;
  char* w = (char*)workspace;
  c.cand_key = (uint32_t*)w;
  c.cand_idx = (int32_t*)(w + slots * kCandCap * sizeof(uint32_t));
  c.cand_cnt = (int32_t*)(w + slots * kCandCap * 2 * sizeof(uint32_t));
  c.arg_val = (float*)(c.cand_cnt + slots);
  c.arg_idx = (int32_t*)(c.arg_val + slots);
  hipLaunchKernelGGL(sample_chunk_kernel, dim3((unsigned)c.chunks, (unsigned)rows), dim3(kCandThreads), 0,
                     (hipStream_t)stream, c);
  hipLaunchKernelGGL(sample_finish_kernel, dim3((unsigned)rows), dim3(kFinishThreads), 0, (hipStream_t)stream, c);
  return check_launch("msa_sample");
}

extern "C" int msa_verify_greedy(const int64_t* target_ids, int64_t batch, int64_t k, const int64_t* drafts,
                                 const int64_t* num_drafts, int64_t* accepted, int64_t* next_token,
                                 msa_stream_t stream) {
  if (batch == 0) return MSA_OK;
  if (!target_ids || !drafts || !num_drafts || !accepted || !next_token)
    return fail(MSA_ERR_INVALID, "msa_verify_greedy: null pointer");
  if (batch < 0 || batch > 0x7fffffff || k < 0 || k > 0x7fffffff) return fail(MSA_ERR_INVALID, "msa_verify_greedy: bad shape");
  hipLaunchKernelGGL(verify_greedy_kernel, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     target_ids, (int)k, drafts, num_drafts, (int)batch, accepted, next_token);
  return check_launch("msa_verify_greedy");
}

extern "C" int msa_verify_sampled(const float* target_probs, int64_t batch, int64_t k, int64_t vocab,
                                  const int64_t* drafts, const int64_t* num_drafts, const float* draft_probs,
                                  const float* uniform, const float* noise, int64_t* accepted, int64_t* next_token,
                                  msa_stream_t stream) {
  if (batch == 0) return MSA_OK;
  if (!target_probs || !drafts || !num_drafts || !uniform || !noise || !accepted || !next_token)
    return fail(MSA_ERR_INVALID, "msa_verify_sampled: null pointer");
  if (batch < 0 || batch > 0x7fffffff || k < 1 || k > 0x7fffffff || vocab <= 0 || vocab > 0x7fffffff)
    return fail(MSA_ERR_INVALID, "msa_verify_sampled: bad shape (k >= 1)");
  hipLaunchKernelGGL(verify_sampled_kernel, dim3((unsigned)batch), dim3(kSampThreads), 0, (hipStream_t)stream,
                     target_probs, (int)k, vocab, drafts, num_drafts, draft_probs, uniform, noise, accepted, next_token);
  return check_launch("msa_verify_sampled");
}
