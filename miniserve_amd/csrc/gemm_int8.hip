// Int8 weight-only linear for prefill-sized batches (M >= 128 tokens): an LDS-tiled MFMA GEMM.
//
// y[m, n] = sum_k x[m, k] * bf16(q[n, k] * s[n]) with float32 accumulation, as Int8Linear.forward
// (quant/int8.py:35-37) computes it, but the int8 weights are dequantized once per 128 x 64 tile
// into LDS instead of materializing the whole bf16 matrix.
//
//  * Workgroup = 4 wavefronts (2 x 2) owning a 128-token x 128-weight-row output tile; a wavefront
//    owns 64 x 64 = 4 x 4 tiles of v_mfma_f32_16x16x32_bf16 (tokens as the A rows, weight rows as
//    the B columns).
//  * Per 64-wide K step: the workgroup loads the x tile (128 x 64 bf16, 16 KB) and the q tile
//    (128 x 64 int8, 8 KB) into registers, dequantizes q to bf16(q * s) on the way into LDS, and
//    computes the step from the other LDS buffer (double buffered: the next step's global loads
//    are in flight during the MFMAs).
//  * Epilogues: bf16 store; residual add (in place allowed); silu(gate) * up, with the tile's
//    weight rows laid out so that every gate column and its up column land in the same lane.
#include <hip/hip_runtime.h>

#include "common.h"

namespace msa {

constexpr int kGBM = 128, kGBN = 128, kGBK = 64;
constexpr int kGLd = kGBK + 8;  // bf16 elements per LDS row (16 bytes of padding)
constexpr size_t kGemmLds = 2 * (size_t)(kGBM + kGBN) * kGLd * 2;

struct GemmArgs {
  const uint16_t* x;
  int64_t ldx;
  const int8_t* w;
  const uint16_t* scale;
  uint16_t* y;
  int64_t ldy;
  const uint16_t* resid;
  int64_t ldr;
  int m, n, k;
  int n_blocks;  // weight-row blocks (of 128 rows, or 64 gate + 64 up for SILU_MUL)
};

__device__ __forceinline__ bf16x8 gemm_dequant8(uint32_t lo, uint32_t hi, float s) {
  bf16x8 r;
  r[0] = (__bf16)((float)(signed char)(lo) * s);
  r[1] = (__bf16)((float)(signed char)(lo >> 8) * s);
  r[2] = (__bf16)((float)(signed char)(lo >> 16) * s);
  r[3] = (__bf16)((float)(signed char)(lo >> 24) * s);
  r[4] = (__bf16)((float)(signed char)(hi) * s);
  r[5] = (__bf16)((float)(signed char)(hi >> 8) * s);
  r[6] = (__bf16)((float)(signed char)(hi >> 16) * s);
  r[7] = (__bf16)((float)(signed char)(hi >> 24) * s);
  return r;
}

// Weight row held in LDS row r (0..127) of row block nb.
template <int EPI>
__device__ __forceinline__ int gemm_wrow(const GemmArgs& a, int nb, int r) {
  if constexpr (EPI == MSA_EPI_SILU_MUL) {
    // quarters of 32 rows: gate, up, gate, up -- wavefront column wn owns quarters 2wn, 2wn+1
    const int q = r >> 5, i = r & 31;
    return ((q & 1) ? a.n / 2 : 0) + nb * 64 + (q >> 1) * 32 + i;
  } else {
    return nb * kGBN + r;
  }
}

template <int EPI>
__global__ __launch_bounds__(256) void int8_gemm_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t gsm[];
  uint16_t* As = gsm;                    // [2][128][kGLd]
  uint16_t* Bs = gsm + 2 * kGBM * kGLd;  // [2][128][kGLd]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int nb = blockIdx.x % a.n_blocks, mb = blockIdx.x / a.n_blocks;
  const int m0 = mb * kGBM;

  // Loader roles. A: rows tid/8 + 32i (i < 4), 8-element chunk tid%8. B: rows tid/4 + 64i (i < 2),
  // 16-element chunk tid%4.
  const int ar = tid >> 3, ac = (tid & 7) * 8;
  const uint16_t* ap[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int row = m0 + ar + 32 * i;
    row = row < a.m ? row : a.m - 1;  // rows past m repeat row m-1; their outputs are dropped
    ap[i] = a.x + (int64_t)row * a.ldx + ac;
  }
  const int br = tid >> 2, bc = (tid & 3) * 16;
  const int8_t* bp[2];
  float bs[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int row = gemm_wrow<EPI>(a, nb, br + 64 * i);
    row = row < a.n ? row : a.n - 1;
    bp[i] = a.w + (int64_t)row * a.k + bc;
    bs[i] = bf16_to_f32(a.scale[row]);
  }
  uint4 ra0, ra1, ra2, ra3, rb0, rb1;  // the next K step's tiles, in flight during the MFMAs
#define MSA_GEMM_LOAD(k0)                                   \
  do {                                                      \
    ra0 = *(const uint4*)(ap[0] + (k0));                    \
    ra1 = *(const uint4*)(ap[1] + (k0));                    \
    ra2 = *(const uint4*)(ap[2] + (k0));                    \
    ra3 = *(const uint4*)(ap[3] + (k0));                    \
    rb0 = *(const uint4*)(bp[0] + (k0));                    \
    rb1 = *(const uint4*)(bp[1] + (k0));                    \
  } while (0)
#define MSA_GEMM_STORE(buf)                                                           \
  do {                                                                                \
    uint16_t* A_ = As + (buf) * kGBM * kGLd + ar * kGLd + ac;                         \
    *(uint4*)(A_) = ra0;                                                              \
    *(uint4*)(A_ + 32 * kGLd) = ra1;                                                  \
    *(uint4*)(A_ + 64 * kGLd) = ra2;                                                  \
    *(uint4*)(A_ + 96 * kGLd) = ra3;                                                  \
    uint16_t* B_ = Bs + (buf) * kGBN * kGLd + br * kGLd + bc;                         \
    *(bf16x8*)(B_) = gemm_dequant8(rb0.x, rb0.y, bs[0]);                              \
    *(bf16x8*)(B_ + 8) = gemm_dequant8(rb0.z, rb0.w, bs[0]);                          \
    *(bf16x8*)(B_ + 64 * kGLd) = gemm_dequant8(rb1.x, rb1.y, bs[1]);                  \
    *(bf16x8*)(B_ + 64 * kGLd + 8) = gemm_dequant8(rb1.z, rb1.w, bs[1]);              \
  } while (0)

  f32x4 acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = a.k / kGBK;
  MSA_GEMM_LOAD(0);
  MSA_GEMM_STORE(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) MSA_GEMM_LOAD((kt + 1) * kGBK);
    const uint16_t* A = As + cur * kGBM * kGLd + (wm * 64 + j) * kGLd + g * 8;
    const uint16_t* B = Bs + cur * kGBN * kGLd + (wn * 64 + j) * kGLd + g * 8;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 af[4], bfr[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        af[t] = *(const bf16x8*)(A + t * 16 * kGLd + ks * 32);
        bfr[t] = *(const bf16x8*)(B + t * 16 * kGLd + ks * 32);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfr[nt], acc[mt][nt], 0, 0, 0);
    }
    if (more) MSA_GEMM_STORE(cur ^ 1);
    __syncthreads();
  }
#undef MSA_GEMM_LOAD
#undef MSA_GEMM_STORE

  // lane (g, j) of tile (mt, nt): tokens m0 + wm*64 + mt*16 + 4g + i, LDS weight row wn*64 + nt*16 + j
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = m0 + wm * 64 + mt * 16 + 4 * g + i;
      if (tok >= a.m) continue;
      if constexpr (EPI == MSA_EPI_SILU_MUL) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int col = nb * 64 + wn * 32 + nt * 16 + j;
          if (col >= a.n / 2) continue;
          const float gt = round_bf16(acc[mt][nt][i]), up = round_bf16(acc[mt][nt + 2][i]);
          a.y[(int64_t)tok * a.ldy + col] = f32_to_bf16(round_bf16(gt / (1.0f + expf(-gt))) * up);
        }
      } else {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const int col = nb * kGBN + wn * 64 + nt * 16 + j;
          if (col >= a.n) continue;
          float v = round_bf16(acc[mt][nt][i]);
          if constexpr (EPI == MSA_EPI_RESIDUAL) v += bf16_to_f32(a.resid[(int64_t)tok * a.ldr + col]);
          a.y[(int64_t)tok * a.ldy + col] = f32_to_bf16(v);
        }
      }
    }
}

template <int EPI>
static int launch_gemm(const GemmArgs& a, int blocks, hipStream_t s) {
  static bool attr_set = false;  // the dynamic-LDS limit is a per-kernel attribute, set once
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)int8_gemm_kernel<EPI>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLds);
    if (e != hipSuccess) return fail(MSA_ERR_LAUNCH, std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
    attr_set = true;
  }
  hipLaunchKernelGGL(int8_gemm_kernel<EPI>, dim3(blocks), dim3(256), kGemmLds, s, a);
  return MSA_OK;
}

}  // namespace msa

using namespace msa;

extern "C" int msa_int8_gemm(const uint16_t* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qweight,
                             const uint16_t* scale, int64_t n, uint16_t* y, int64_t ldy, int epilogue,
                             const uint16_t* residual, int64_t ldr, msa_stream_t stream) {
  if (m == 0) return MSA_OK;
  if (!x || !qweight || !scale || !y) return fail(MSA_ERR_INVALID, "msa_int8_gemm: null pointer");
  if (m < 0 || n <= 0 || k <= 0 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
    return fail(MSA_ERR_INVALID, "msa_int8_gemm: bad shape");
  if (k % kGBK != 0) return fail(MSA_ERR_UNSUPPORTED, "msa_int8_gemm: in_features must be a multiple of 64");
  if (ldx < k || ldx % 8 != 0 || !aligned16(x) || !aligned16(qweight))
    return fail(MSA_ERR_INVALID, "msa_int8_gemm: x / qweight must be 16-byte aligned with ldx % 8 == 0");
  if (epilogue < 0 || epilogue > 2) return fail(MSA_ERR_INVALID, "msa_int8_gemm: unknown epilogue");
  if (epilogue == MSA_EPI_SILU_MUL && n % 2 != 0) return fail(MSA_ERR_INVALID, "msa_int8_gemm: SILU_MUL needs an even n");
  const int64_t out_cols = epilogue == MSA_EPI_SILU_MUL ? n / 2 : n;
  if (ldy < out_cols) return fail(MSA_ERR_INVALID, "msa_int8_gemm: ldy too small");
  if (epilogue == MSA_EPI_RESIDUAL && (!residual || ldr < n))
    return fail(MSA_ERR_INVALID, "msa_int8_gemm: the residual epilogue needs residual with ldr >= n");
  GemmArgs a{};
  a.x = x; a.ldx = ldx; a.w = qweight; a.scale = scale; a.y = y; a.ldy = ldy; a.resid = residual; a.ldr = ldr;
  a.m = (int)m; a.n = (int)n; a.k = (int)k;
  a.n_blocks = (int)(epilogue == MSA_EPI_SILU_MUL ? (n / 2 + 63) / 64 : (n + kGBN - 1) / kGBN);
  const int64_t blocks = (int64_t)a.n_blocks * ((m + kGBM - 1) / kGBM);
  if (blocks > 0x7fffffff) return fail(MSA_ERR_INVALID, "msa_int8_gemm: too many tiles");
  hipStream_t s = (hipStream_t)stream;
  int rc;
  switch (epilogue) {
    case MSA_EPI_NONE: rc = launch_gemm<MSA_EPI_NONE>(a, (int)blocks, s); break;
    case MSA_EPI_SILU_MUL: rc = launch_gemm<MSA_EPI_SILU_MUL>(a, (int)blocks, s); break;
    default: rc = launch_gemm<MSA_EPI_RESIDUAL>(a, (int)blocks, s); break;
  }
  if (rc != MSA_OK) return rc;
  return check_launch("msa_int8_gemm");
}
