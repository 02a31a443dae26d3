// Streaming int8 linear for decode batches of up to 16 tokens over large weight matrices (tens to
// hundreds of megabytes): the regime where one launch can keep HBM busy.
//
// A workgroup of eight wavefronts owns a contiguous run of U output units (one workgroup per CU).
// A unit is one 16-row weight tile; for the SiLU epilogue it is 8 gate rows and the 8 matching up
// rows, so the pair meets in one MFMA tile and every workgroup gets the same number of units.
// Wavefront ks owns the ks-th of eight equal K slices of every unit:
//
//  1. Prologue: the norm weights (staged once in LDS), the 16 token rows of activations as
//     contiguous 16-byte pieces (staged in LDS, then read back as the A operand of
//     v_mfma_f32_16x16x32_bf16 for the wavefront's K slice and held in registers for the whole
//     launch), then the first unit's weight fragments. With a norm the wavefronts' partial sums
//     of squares meet in LDS, and each lane rounds its fragments to bf16(w * bf16(x * r)) --
//     model/layers.py:18-22 -- chunk by chunk inside the first unit.
//  2. Per unit, per 64-wide K chunk: the lane's 16 weight bytes (row j, K offsets [16g, 16g + 16))
//     are dequantized to bf16(q * s) -- the value of the reference's whole-matrix dequantization
//     (quant/int8.py:36) -- fed to two MFMAs, and the same registers are refilled at once with the
//     next unit's bytes, so one unit per wavefront is in flight while one is multiplied.
//  3. The eight partial 16 x 16 tiles meet in a double-buffered LDS slot (one barrier per unit);
//     one wavefront, in turn, sums them in a fixed order and rounds them -- bf16(x @ W^T), or
//     bf16(silu(gate) * up) with the reference's rounding points (model/layers.py:77-78) -- into
//     an LDS copy of the workgroup's outputs.
//  4. The outputs leave LDS as one contiguous run of columns per token row (the residual of
//     model/qwen3.py:121-122, read the same way, is added there).
//
// Loads are unconditional (indices clamped) and the unit loop is unrolled, so the compiler's
// in-order load counter waits for exactly the data about to be used.
#include <hip/hip_runtime.h>

#include "common.h"

namespace msa {

enum { ST_PRO_NONE = 0, ST_PRO_RMSNORM = 1 };
enum { ST_EPI_NONE = 0, ST_EPI_SILU_MUL = 1, ST_EPI_RESIDUAL = 2 };

struct StreamArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* norm_w;
  float eps;
  int t;  // tokens, 1..16
  int k;  // in features = 8 * CW * 64
  const int8_t* w;
  const uint16_t* scale;
  int n;      // weight rows ([gate | up] for SILU_MUL)
  int units;  // output units
  uint16_t* y;
  int64_t ldy;
  const uint16_t* resid;
  int64_t ldr;
};

constexpr int kStreamWaves = 8;
constexpr int kStreamMaxUnits = 8;  // units per workgroup (unrolled; their outputs wait in LDS)

// Weight row of unit u for lane row j (clamped into the matrix; outputs past the end are dropped).
template <int EPI>
__device__ __forceinline__ int stream_row(const StreamArgs& a, int u, int j) {
  if constexpr (EPI == ST_EPI_SILU_MUL) {
    const int half = a.n / 2;
    return min(8 * u + (j & 7), half - 1) + (j < 8 ? 0 : half);
  } else {
    return min(16 * u + j, a.n - 1);
  }
}

// CW 64-wide K chunks per wavefront (k = 8 * CW * 64); U units per workgroup.
template <int CW, int U, int PRO, int EPI>
__global__ __launch_bounds__(64 * kStreamWaves) void dec_stream_kernel(StreamArgs a) {
  constexpr int W = kStreamWaves;
  static_assert(U >= 1 && U <= kStreamMaxUnits, "unit run");
  constexpr bool NORM = PRO == ST_PRO_RMSNORM;
  constexpr int KS = CW * 64;                           // K elements per wavefront
  constexpr int UC = EPI == ST_EPI_SILU_MUL ? 8 : 16;  // output columns per unit
  constexpr int XPITCH = W * KS + 8;                    // staged activation row pitch (elements)
  __shared__ f32x4 s_red[2][W][64];
  __shared__ float s_ss[W][16];
  __shared__ __attribute__((aligned(16))) uint16_t s_nw[NORM ? W * KS : 8];
  __shared__ __attribute__((aligned(16))) uint16_t s_x[16 * XPITCH];
  __shared__ uint16_t s_out[16][U * UC];  // [token][column of the run]

  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wavefront-uniform: scalar branches
  const int j = lane & 15, g = lane >> 4;
  const int ubase = blockIdx.x * U;
  const int ulast = min(ubase + U, a.units) - 1;  // this workgroup's last unit
  const int koff = ks * KS + g * 16;              // this lane's first K element in every chunk

  // ---- 1. the norm weights, the activations, then the first unit's scale and weights ----
  // Loads complete in issue order, so each group is requested before everything that is needed
  // after it: waiting for the activations does not wait for the weights.
  // At most two 16-byte pieces of the norm weights per thread (k <= 8192); piece indices are
  // clamped, so surplus threads repeat the last piece.
  constexpr int NWPIECES = W * KS / 8;
  static_assert(!NORM || NWPIECES <= 2 * 64 * W, "norm weights: two pieces per thread");
  const int nwi0 = min((int)threadIdx.x, NWPIECES - 1), nwi1 = min(64 * W + (int)threadIdx.x, NWPIECES - 1);
  uint4 nw0{}, nw1{};
  if constexpr (NORM) {
    nw0 = *(const uint4*)(a.norm_w + nwi0 * 8);
    if constexpr (NWPIECES > 64 * W) nw1 = *(const uint4*)(a.norm_w + nwi1 * 8);
  }
  // The activations: 16 rows (rows past t repeat row t - 1) of RP contiguous 16-byte pieces,
  // 2 * CW per thread, held in the fragment registers until they are staged.
  uint4 xa[CW][2];
  constexpr int RP = W * KS / 8;
#pragma unroll
  for (int q = 0; q < 2 * CW; ++q) {
    const int pc = q * 64 * W + (int)threadIdx.x, row = pc / RP, col = pc % RP;
    xa[q >> 1][q & 1] = *(const uint4*)(a.x + (int64_t)min(row, a.t - 1) * a.ldx + col * 8);
  }
  __builtin_amdgcn_sched_barrier(0);  // the activations stay ahead of the weight loads
  uint4 wv[CW];
  uint32_t scb;
  {
    const int row = stream_row<EPI>(a, min(ubase, ulast), j);
    scb = a.scale[row];
    const int8_t* p = a.w + (int64_t)row * a.k + koff;
#pragma unroll
    for (int c = 0; c < CW; ++c) wv[c] = *(const uint4*)(p + c * 64);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the first wait
#pragma unroll
  for (int q = 0; q < 2 * CW; ++q) {
    const int pc = q * 64 * W + (int)threadIdx.x, row = pc / RP, col = pc % RP;
    *(uint4*)(s_x + row * XPITCH + col * 8) = xa[q >> 1][q & 1];
  }
  if constexpr (NORM) {
    *(uint4*)(s_nw + nwi0 * 8) = nw0;
    if constexpr (NWPIECES > 64 * W) *(uint4*)(s_nw + nwi1 * 8) = nw1;
  }
  __syncthreads();  // the staged activations and norm weights
#pragma unroll
  for (int c = 0; c < CW; ++c) {
    xa[c][0] = *(const uint4*)(s_x + j * XPITCH + koff + c * 64);
    xa[c][1] = *(const uint4*)(s_x + j * XPITCH + koff + c * 64 + 8);
  }
  float rn = 0.f;  // this lane's token's 1 / rms (with a norm)
  if constexpr (NORM) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CW; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        s = dot2_bf16(xa[c][h].x, xa[c][h].x, s);
        s = dot2_bf16(xa[c][h].y, xa[c][h].y, s);
        s = dot2_bf16(xa[c][h].z, xa[c][h].z, s);
        s = dot2_bf16(xa[c][h].w, xa[c][h].w, s);
      }
    s = xrow_sum(s);
    if (g == 0) s_ss[ks][j] = s;
    __syncthreads();  // every wavefront's partial sums of squares
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) tot += s_ss[w][j];
    rn = 1.0f / sqrtf(tot / (float)a.k + a.eps);
  }
  __builtin_amdgcn_sched_barrier(0);  // nothing of the unit loop (which waits for weights) moves up here

  // ---- 2./3. the workgroup's units ----
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const bool refill = i + 1 < U;  // a compile-time fact after unrolling
    const float sf = bf16_to_f32(scb);
    const int8_t* pn = a.w;
    if (refill) {
      const int rown = stream_row<EPI>(a, min(ubase + i + 1, ulast), j);
      scb = a.scale[rown];  // requested before the refill: waited for with the next unit
      pn = a.w + (int64_t)rown * a.k + koff;
    }
    // Four independent accumulation chains (chunk parity x k-step).
    f32x4 acc4[4] = {};
#pragma unroll
    for (int c = 0; c < CW; ++c) {
      if (NORM && i == 0) {
        // The norm is applied chunk by chunk inside the first unit, so the next unit's refills
        // start as soon as the sums of squares are known.
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint4 wn = *(const uint4*)(s_nw + koff + c * 64 + h * 8);
          uint4& v = xa[c][h];
          v = uint4{norm_pair(v.x, wn.x & 0xffffu, wn.x & 0xffff0000u, rn),
                    norm_pair(v.y, wn.y & 0xffffu, wn.y & 0xffff0000u, rn),
                    norm_pair(v.z, wn.z & 0xffffu, wn.z & 0xffff0000u, rn),
                    norm_pair(v.w, wn.w & 0xffffu, wn.w & 0xffff0000u, rn)};
        }
      }
      const bf16x8 b0 = dequant8(wv[c].x, wv[c].y, sf);
      const bf16x8 b1 = dequant8(wv[c].z, wv[c].w, sf);
      if (refill) wv[c] = *(const uint4*)(pn + c * 64);
      // Pinned here: left to itself the scheduler sinks the refills below the last MFMA, and the
      // wavefront then has less in flight while it multiplies.
      __builtin_amdgcn_sched_barrier(0);
      f32x4& a0 = acc4[(c & 1) * 2];
      f32x4& a1 = acc4[(c & 1) * 2 + 1];
      a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[c][0]), b0, a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[c][1]), b1, a1, 0, 0, 0);
    }
    s_red[i & 1][ks][lane] = (acc4[0] + acc4[1]) + (acc4[2] + acc4[3]);
    __syncthreads();
    if (ks == i % W) {
      // Lane (j, g) holds output rows 4g..4g+3 (tokens) of tile column j (weight row j); the
      // results wait in LDS, so no store joins the loads in the in-order counter.
      f32x4 v = s_red[i & 1][0][lane];
#pragma unroll
      for (int w = 1; w < W; ++w) v += s_red[i & 1][w][lane];
      if constexpr (EPI == ST_EPI_SILU_MUL) {
        f32x4 up;
#pragma unroll
        for (int q = 0; q < 4; ++q) up[q] = __shfl_xor(v[q], 8);
        if (j < 8) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gt = round_bf16(v[q]), upv = round_bf16(up[q]);
            s_out[4 * g + q][i * UC + j] = f32_to_bf16(round_bf16(silu_f32(gt)) * upv);
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) s_out[4 * g + q][i * UC + j] = f32_to_bf16(v[q]);
      }
    }
  }

  // ---- 4. the workgroup's outputs: a contiguous run of columns per token row ----
  __syncthreads();
  const int c0 = ubase * UC;
  const int ncols = min(U * UC, (EPI == ST_EPI_SILU_MUL ? a.n / 2 : a.n) - c0);
  for (int e = threadIdx.x; e < a.t * ncols; e += 64 * W) {
    const int tk = e / ncols, cc = e - tk * ncols;
    uint16_t o = s_out[tk][cc];
    // bf16(residual + bf16(x @ W^T)); the residual is read just before y is written (it may be y).
    if constexpr (EPI == ST_EPI_RESIDUAL) o = f32_to_bf16(bf16_to_f32(o) + bf16_to_f32(a.resid[(int64_t)tk * a.ldr + c0 + cc]));
    a.y[(int64_t)tk * a.ldy + c0 + cc] = o;
  }
}

// ---- host side ----------------------------------------------------------------------------------

// Streaming pays off once every CU has at least one and a half units to stream (with fewer, the
// per-workgroup prologue -- 16 x k activations through LDS and the norm -- dominates).
constexpr int kStreamMinUnits = 384;

static int stream_cw(int64_t k) { return (k == 2048 || k == 4096) ? (int)(k / (64 * kStreamWaves)) : 0; }

bool dec_stream_eligible(int64_t m, int64_t k, int64_t n, int epilogue) {
  if (m < 1 || m > 16 || stream_cw(k) == 0) return false;
  const int64_t units = epilogue == ST_EPI_SILU_MUL ? (n / 2 + 7) / 8 : (n + 15) / 16;
  return units >= kStreamMinUnits;
}

template <int CW, int U, int PRO, int EPI>
static void stream_launch(const StreamArgs& a, hipStream_t s) {
  const int grid = (a.units + U - 1) / U;
  hipLaunchKernelGGL((dec_stream_kernel<CW, U, PRO, EPI>), dim3(grid), dim3(64 * kStreamWaves), 0, s, a);
}

// Units per workgroup: enough for one workgroup per CU (256 CUs), at most kStreamMaxUnits.
template <int CW, int PRO, int EPI>
static int stream_dispatch_u(const StreamArgs& a, hipStream_t s) {
  const int u = (a.units + 255) / 256;
  switch (u) {
    case 1: stream_launch<CW, 1, PRO, EPI>(a, s); break;
    case 2: stream_launch<CW, 2, PRO, EPI>(a, s); break;
    case 3: stream_launch<CW, 3, PRO, EPI>(a, s); break;
    case 4: stream_launch<CW, 4, PRO, EPI>(a, s); break;
    case 5:
    case 6: stream_launch<CW, 6, PRO, EPI>(a, s); break;
    default: stream_launch<CW, 8, PRO, EPI>(a, s); break;
  }
  return MSA_OK;
}

template <int PRO, int EPI>
static int stream_dispatch(const StreamArgs& a, hipStream_t s) {
  return stream_cw(a.k) == 4 ? stream_dispatch_u<4, PRO, EPI>(a, s) : stream_dispatch_u<8, PRO, EPI>(a, s);
}

int launch_dec_stream(const uint16_t* x, int64_t ldx, int64_t m, int64_t k, const uint16_t* norm_w, float eps,
                      const int8_t* qweight, const uint16_t* scale, int64_t n, int epilogue, uint16_t* y, int64_t ldy,
                      const uint16_t* residual, int64_t ldr, hipStream_t s) {
  if (!dec_stream_eligible(m, k, n, epilogue)) return fail(MSA_ERR_UNSUPPORTED, "streaming linear: shape not eligible");
  StreamArgs a{};
  a.x = x; a.ldx = ldx; a.norm_w = norm_w; a.eps = eps; a.t = (int)m; a.k = (int)k; a.w = qweight; a.scale = scale;
  a.n = (int)n; a.y = y; a.ldy = ldy; a.resid = residual; a.ldr = ldr;
  a.units = (int)(epilogue == ST_EPI_SILU_MUL ? (n / 2 + 7) / 8 : (n + 15) / 16);
  const bool nrm = norm_w != nullptr;
  int rc;
  if (epilogue == ST_EPI_SILU_MUL) {
    rc = nrm ? stream_dispatch<ST_PRO_RMSNORM, ST_EPI_SILU_MUL>(a, s) : stream_dispatch<ST_PRO_NONE, ST_EPI_SILU_MUL>(a, s);
  } else if (epilogue == ST_EPI_RESIDUAL) {
    if (nrm) return fail(MSA_ERR_UNSUPPORTED, "streaming linear: the residual epilogue takes no norm");
    rc = stream_dispatch<ST_PRO_NONE, ST_EPI_RESIDUAL>(a, s);
  } else if (epilogue == ST_EPI_NONE) {
    rc = nrm ? stream_dispatch<ST_PRO_RMSNORM, ST_EPI_NONE>(a, s) : stream_dispatch<ST_PRO_NONE, ST_EPI_NONE>(a, s);
  } else {
    return fail(MSA_ERR_INVALID, "streaming linear: unknown epilogue");
  }
  if (rc != MSA_OK) return rc;
  return check_launch("streaming linear");
}

}  // namespace msa
