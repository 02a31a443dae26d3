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
  for (int w = 1; w < kSampWaves; ++w) r = fmaxf(r, sh.fred[w]);
  return r;
}

__device__ __forceinline__ float block_sum(float v, SampShared& sh) {
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = 0.f;
  for (int w = 0; w < kSampWaves; ++w) r += sh.fred[w];  // fixed order
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
  for (int w = 1; w < kSampWaves; ++w)
    if (sh.fred[w] > bv || (sh.fred[w] == bv && sh.ired[w] < bi)) {
      bv = sh.fred[w];
      bi = sh.ired[w];
    }
  return bi;
}

__global__ __launch_bounds__(kSampThreads) void sample_rows_kernel(SampArgs a) {
  __shared__ SampShared sh;
  const int64_t row = blockIdx.x;
  const float* lg = a.logits + row * a.ld;
  const int64_t V = a.vocab;
  const int tid = threadIdx.x;

  if (a.mode == SAMP_SAMPLE && a.greedy && a.greedy[row]) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int64_t i = tid; i < V; i += kSampThreads) {
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
  for (int64_t i = tid; i < V; i += kSampThreads) mloc = fmaxf(mloc, lg[i] / t);
  const float m = block_max(mloc, sh);

  // ---- top-k: key of the k-th largest z -----------------------------------------------------
  uint32_t kmin = 0;  // keep z with ord_key(z) >= kmin
  const int64_t k = a.top_k ? a.top_k[row] : 0;
  if (k > 0 && k < V) {
    uint32_t prefix = 0, pmask = 0;
    int64_t remaining = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int b = tid; b < 256; b += kSampThreads) sh.hist.cnt[b] = 0;
      __syncthreads();
      for (int64_t i = tid; i < V; i += kSampThreads) {
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
    for (int64_t i = tid; i < V; i += kSampThreads) {
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
      for (int b = tid; b < 256; b += kSampThreads) sh.hist.mass[b] = 0ull;
      __syncthreads();
      for (int64_t i = tid; i < V; i += kSampThreads) {
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
    for (int64_t i = tid; i < V; i += kSampThreads) {
      const float z = lg[i] / t;
      o[i] = ord_key(z) >= cut ? z : -INFINITY;
    }
    return;
  }
  float zl = 0.f;
  for (int64_t i = tid; i < V; i += kSampThreads) {
    const float z = lg[i] / t;
    if (ord_key(z) >= cut) zl += expf(z - m);
  }
  const float zsum = block_sum(zl, sh);
  if (a.mode == SAMP_PROBS) {
    float* o = a.out + row * a.ldo;
    for (int64_t i = tid; i < V; i += kSampThreads) {
      const float z = lg[i] / t;
      o[i] = ord_key(z) >= cut ? expf(z - m) / zsum : 0.f;
    }
    return;
  }
  const float* nz = a.noise + row * a.ldn;
  float bv = -1.f;
  int bi = 0x7fffffff;
  for (int64_t i = tid; i < V; i += kSampThreads) {
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

extern "C" int msa_sample(const float* logits, int64_t ld, int64_t rows, int64_t vocab, const float* temperature,
                          const int32_t* top_k, const float* top_p, const uint8_t* greedy, const float* noise,
                          int64_t ldn, int64_t* out_ids, msa_stream_t stream) {
  if (!out_ids || !noise || ldn < vocab) return fail(MSA_ERR_INVALID, "msa_sample: bad noise / out_ids");
  SampArgs a{};
  a.logits = logits; a.ld = ld; a.vocab = vocab; a.temperature = temperature; a.top_k = top_k; a.top_p = top_p;
  a.greedy = greedy; a.noise = noise; a.ldn = ldn; a.ids = out_ids; a.mode = SAMP_SAMPLE;
  return sample_launch(a, rows, (hipStream_t)stream, "msa_sample");
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
