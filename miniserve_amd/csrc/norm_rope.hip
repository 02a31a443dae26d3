// RMSNorm, residual add + RMSNorm, and the fused per-head q/k RMSNorm + RoPE + KV-cache write.
//
// Rounding follows the reference's bf16 op sequence, so that these kernels agree with it to the
// bit except for the order of the float32 sum of squares:
//  * RMSNorm (model/layers.py:19-22): x32 * rsqrt(mean(x32^2) + eps) is rounded to bf16 BEFORE the
//    bf16 weight multiply, whose product is rounded again.
//  * residual add (model/qwen3.py:121-122): bf16 + bf16 rounded to bf16.
//  * RoPE (model/layers.py:61-65): cos/sin rounded to bf16; q*cos and rotate_half(q)*sin are each
//    rounded to bf16, then their sum is rounded.
// One wavefront per row (or per (token, head)); a workgroup holds four.
#include "common.h"

namespace msa {

__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                      const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                                      int64_t ldo, int64_t rows, int dim, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const uint16_t* xr = x + row * ldx;
  float ss = 0.f;
  for (int c = lane * 8; c < dim; c += 512) {
    const uint4 v = *(const uint4*)(xr + c);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = bf16lo(u[e]), b = bf16hi(u[e]);
      ss += a * a + b * b;
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)dim + eps);
  uint16_t* orow = out + row * ldo;
  for (int c = lane * 8; c < dim; c += 512) {
    const uint4 v = *(const uint4*)(xr + c);
    const uint4 wv = *(const uint4*)(w + c);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = round_bf16(bf16lo(u[e]) * r), b = round_bf16(bf16hi(u[e]) * r);
      o[e] = pack_bf16x2(bf16lo(ww[e]) * a, bf16hi(ww[e]) * b);
    }
    *(uint4*)(orow + c) = uint4{o[0], o[1], o[2], o[3]};
  }
}

__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const uint16_t* resid_in, const uint16_t* __restrict__ delta,
                                                          uint16_t* resid_out, const uint16_t* __restrict__ w,
                                                          uint16_t* __restrict__ out, int64_t rows, int dim, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const uint16_t* ri = resid_in + row * dim;
  uint16_t* rr = resid_out + row * dim;
  const uint16_t* dr = delta + row * dim;
  float ss = 0.f;
  for (int c = lane * 8; c < dim; c += 512) {
    const uint4 a = *(const uint4*)(ri + c);
    const uint4 d = *(const uint4*)(dr + c);
    const uint32_t ua[4] = {a.x, a.y, a.z, a.w}, ud[4] = {d.x, d.y, d.z, d.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = round_bf16(bf16lo(ua[e]) + bf16lo(ud[e]));
      const float hi = round_bf16(bf16hi(ua[e]) + bf16hi(ud[e]));
      ss += lo * lo + hi * hi;
      o[e] = pack_bf16x2(lo, hi);
    }
    *(uint4*)(rr + c) = uint4{o[0], o[1], o[2], o[3]};
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)dim + eps);
  uint16_t* orow = out + row * dim;
  for (int c = lane * 8; c < dim; c += 512) {
    const uint4 v = *(const uint4*)(rr + c);  // this lane's own stores above
    const uint4 wv = *(const uint4*)(w + c);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = round_bf16(bf16lo(u[e]) * r), b = round_bf16(bf16hi(u[e]) * r);
      o[e] = pack_bf16x2(bf16lo(ww[e]) * a, bf16hi(ww[e]) * b);
    }
    *(uint4*)(orow + c) = uint4{o[0], o[1], o[2], o[3]};
  }
}

// One wavefront per (token, head slot); head slots are q heads, then k heads, then v heads.
// Lane l owns the RoPE pairs (i, i + D/2) for i = l, l + 64. The qkv row comes either as bf16
// (PARTIAL = false) or as k_split float32 split-K partials of the qkv projection, summed here in
// split order and rounded to bf16 -- the value the projection would have produced.
template <bool PARTIAL>
__global__ __launch_bounds__(256) void qk_norm_rope_cache_kernel(
    const uint16_t* __restrict__ qkv, int64_t ldqkv, const float* __restrict__ part, int k_split, int64_t tokens,
    int heads, int kv_heads, int dim, const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw, float eps,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, const int64_t* __restrict__ slots,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, int64_t num_slots) {
  const int slots_per_tok = heads + 2 * kv_heads;
  const int64_t idx = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (idx >= tokens * slots_per_tok) return;
  const int lane = threadIdx.x & 63;
  const int64_t t = idx / slots_per_tok;
  const int hs = (int)(idx % slots_per_tok);
  const int64_t row_cols = (int64_t)slots_per_tok * dim;
  const uint16_t* src = qkv + t * ldqkv + (int64_t)hs * dim;
  const float* psrc = part + t * row_cols + (int64_t)hs * dim;
  const int64_t pstride = tokens * row_cols;
  auto load = [&](int i) -> float {
    if constexpr (PARTIAL) {
      float acc = 0.f;
      for (int s = 0; s < k_split; ++s) acc += psrc[s * pstride + i];
      return round_bf16(acc);
    } else {
      return bf16_to_f32(src[i]);
    }
  };
  const int half = dim / 2;
  if (hs >= heads + kv_heads) {
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) return;
    uint16_t* dst = v_cache + (slot * kv_heads + (hs - heads - kv_heads)) * dim;
    for (int i = lane; i < dim; i += 64) dst[i] = f32_to_bf16(load(i));
    return;
  }
  const bool is_q = hs < heads;
  uint16_t* dst;
  if (is_q) {
    dst = q_out + (t * heads + hs) * dim;
  } else {
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) return;  // the whole wave leaves together
    dst = k_cache + (slot * kv_heads + (hs - heads)) * dim;
  }
  const uint16_t* nw = is_q ? qw : kw;
  float lo[2] = {0.f, 0.f}, hi[2] = {0.f, 0.f};
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int i = lane + 64 * p;
    if (i < half) {
      lo[p] = load(i);
      hi[p] = load(i + half);
      ss += lo[p] * lo[p] + hi[p] * hi[p];
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)dim + eps);
  const float* cr = cos_t + t * dim;
  const float* sr = sin_t + t * dim;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int i = lane + 64 * p;
    if (i < half) {
      const float a = round_bf16(bf16_to_f32(nw[i]) * round_bf16(lo[p] * r));
      const float b = round_bf16(bf16_to_f32(nw[i + half]) * round_bf16(hi[p] * r));
      const float c_lo = round_bf16(cr[i]), c_hi = round_bf16(cr[i + half]);
      const float s_lo = round_bf16(sr[i]), s_hi = round_bf16(sr[i + half]);
      dst[i] = f32_to_bf16(round_bf16(a * c_lo) + round_bf16(-b * s_lo));
      dst[i + half] = f32_to_bf16(round_bf16(b * c_hi) + round_bf16(a * s_hi));
    }
  }
}

// The same op for head_dim 128 with 16-byte accesses: one workgroup per (token, 32 head slots),
// eight threads per head slot. Thread (slot, sub) holds dims [8 sub, 8 sub + 8) and their RoPE
// partners [64 + 8 sub, 64 + 8 sub + 8), so every rotation pair is in one thread; the head's sum of
// squares meets over the eight threads. All loads of a thread are issued before any use: one
// memory round trip per token instead of one per dependent step.
template <bool PARTIAL>
__global__ __launch_bounds__(256) void qk_norm_rope_cache_d128_kernel(
    const uint16_t* __restrict__ qkv, int64_t ldqkv, const float* __restrict__ part, int k_split, int64_t tokens,
    int heads, int kv_heads, const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw, float eps,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, const int64_t* __restrict__ slots,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, int64_t num_slots) {
  constexpr int D = 128;
  const int nslots = heads + 2 * kv_heads;
  const int groups = (nslots + 31) / 32;
  const int64_t t = blockIdx.x / groups;
  const int hs = (int)(blockIdx.x % groups) * 32 + (int)(threadIdx.x >> 3);
  const int sub = threadIdx.x & 7;
  const bool live = hs < nslots;
  const int hsc = live ? hs : nslots - 1;  // idle threads read a real slot and store nothing
  const int d0 = 8 * sub, d1 = 64 + 8 * sub;
  // the head slot's 16 values, as floats (bf16-rounded partial sums for PARTIAL)
  float lo[8], hi[8];
  if constexpr (PARTIAL) {
    const int64_t row_cols = (int64_t)nslots * D, pstride = tokens * row_cols;
    const float* p = part + t * row_cols + (int64_t)hsc * D;
    float4 a0 = *(const float4*)(p + d0), a1 = *(const float4*)(p + d0 + 4);
    float4 b0 = *(const float4*)(p + d1), b1 = *(const float4*)(p + d1 + 4);
    for (int s = 1; s < k_split; ++s) {
      const float* q = p + s * pstride;
      const float4 c0 = *(const float4*)(q + d0), c1 = *(const float4*)(q + d0 + 4);
      const float4 e0 = *(const float4*)(q + d1), e1 = *(const float4*)(q + d1 + 4);
      a0.x += c0.x; a0.y += c0.y; a0.z += c0.z; a0.w += c0.w; a1.x += c1.x; a1.y += c1.y; a1.z += c1.z; a1.w += c1.w;
      b0.x += e0.x; b0.y += e0.y; b0.z += e0.z; b0.w += e0.w; b1.x += e1.x; b1.y += e1.y; b1.z += e1.z; b1.w += e1.w;
    }
    const float la[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float lb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lo[e] = round_bf16(la[e]);
      hi[e] = round_bf16(lb[e]);
    }
  } else {
    const uint16_t* src = qkv + t * ldqkv + (int64_t)hsc * D;
    const uint4 ul = *(const uint4*)(src + d0), uh = *(const uint4*)(src + d1);
    const uint32_t wl[4] = {ul.x, ul.y, ul.z, ul.w}, wh[4] = {uh.x, uh.y, uh.z, uh.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo[2 * e] = bf16lo(wl[e]);
      lo[2 * e + 1] = bf16hi(wl[e]);
      hi[2 * e] = bf16lo(wh[e]);
      hi[2 * e + 1] = bf16hi(wh[e]);
    }
  }
  const bool is_q = hsc < heads, is_v = hsc >= heads + kv_heads;
  const uint16_t* nw = is_q ? qw : kw;
  const uint4 nl = *(const uint4*)(nw + d0), nh = *(const uint4*)(nw + d1);
  const float* cr = cos_t + t * D;
  const float* sr = sin_t + t * D;
  const float4 cl0 = *(const float4*)(cr + d0), cl1 = *(const float4*)(cr + d0 + 4);
  const float4 ch0 = *(const float4*)(cr + d1), ch1 = *(const float4*)(cr + d1 + 4);
  const float4 sl0 = *(const float4*)(sr + d0), sl1 = *(const float4*)(sr + d0 + 4);
  const float4 sh0 = *(const float4*)(sr + d1), sh1 = *(const float4*)(sr + d1 + 4);
  const int64_t slot = slots[t];
  const bool cached = slot >= 0 && slot < num_slots;

  if (is_v) {
    if (live && cached) {
      uint16_t* dst = v_cache + (slot * kv_heads + (hsc - heads - kv_heads)) * D;
      *(uint4*)(dst + d0) = uint4{pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3]), pack_bf16x2(lo[4], lo[5]),
                                  pack_bf16x2(lo[6], lo[7])};
      *(uint4*)(dst + d1) = uint4{pack_bf16x2(hi[0], hi[1]), pack_bf16x2(hi[2], hi[3]), pack_bf16x2(hi[4], hi[5]),
                                  pack_bf16x2(hi[6], hi[7])};
    }
    return;  // the eight threads of a head slot leave together
  }
  const float cl[8] = {cl0.x, cl0.y, cl0.z, cl0.w, cl1.x, cl1.y, cl1.z, cl1.w};
  const float ch[8] = {ch0.x, ch0.y, ch0.z, ch0.w, ch1.x, ch1.y, ch1.z, ch1.w};
  const float sl[8] = {sl0.x, sl0.y, sl0.z, sl0.w, sl1.x, sl1.y, sl1.z, sl1.w};
  const float sh[8] = {sh0.x, sh0.y, sh0.z, sh0.w, sh1.x, sh1.y, sh1.z, sh1.w};
  float ol[8], oh[8];
  head_norm_rope8(lo, hi, nl, nh, cl, ch, sl, sh, eps, ol, oh);
  if (!live || (!is_q && !cached)) return;
  uint16_t* dst = is_q ? q_out + (t * heads + hsc) * D : k_cache + (slot * kv_heads + (hsc - heads)) * D;
  *(uint4*)(dst + d0) = uint4{pack_bf16x2(ol[0], ol[1]), pack_bf16x2(ol[2], ol[3]), pack_bf16x2(ol[4], ol[5]),
                              pack_bf16x2(ol[6], ol[7])};
  *(uint4*)(dst + d1) = uint4{pack_bf16x2(oh[0], oh[1]), pack_bf16x2(oh[2], oh[3]), pack_bf16x2(oh[4], oh[5]),
                              pack_bf16x2(oh[6], oh[7])};
}

// Residual add + RMSNorm whose delta arrives as k_split float32 split-K partials [k_split][rows][dim]
// of the projection before it: delta = bf16(sum of partials in split order), residual_out =
// bf16(residual + delta), out = RMSNorm(residual_out). One workgroup per row.
__global__ __launch_bounds__(256) void splitk_add_rmsnorm_kernel(const float* __restrict__ part, int k_split,
                                                                 int64_t rows, int dim, const uint16_t* resid_in,
                                                                 uint16_t* resid_out, const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ out, float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t stride = rows * dim;
  const float* pr = part + row * dim;
  const uint16_t* ri = resid_in + row * dim;
  uint16_t* ro = resid_out + row * dim;
  float ss = 0.f;
  for (int c = tid * 4; c < dim; c += 1024) {
    float4 acc = *(const float4*)(pr + c);
    for (int s = 1; s < k_split; ++s) {
      const float4 v = *(const float4*)(pr + s * stride + c);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    const uint2 rv = *(const uint2*)(ri + c);
    const float x0 = round_bf16(round_bf16(acc.x) + bf16lo(rv.x));
    const float x1 = round_bf16(round_bf16(acc.y) + bf16hi(rv.x));
    const float x2 = round_bf16(round_bf16(acc.z) + bf16lo(rv.y));
    const float x3 = round_bf16(round_bf16(acc.w) + bf16hi(rv.y));
    ss += x0 * x0 + x1 * x1 + x2 * x2 + x3 * x3;
    *(uint2*)(ro + c) = uint2{pack_bf16x2(x0, x1), pack_bf16x2(x2, x3)};
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  ss = red[0] + red[1] + red[2] + red[3];
  const float r = 1.0f / sqrtf(ss / (float)dim + eps);
  uint16_t* orow = out + row * dim;
  for (int c = tid * 4; c < dim; c += 1024) {
    const uint2 v = *(const uint2*)(ro + c);  // this thread's own stores above
    const uint2 wv = *(const uint2*)(w + c);
    const float a0 = round_bf16(bf16lo(v.x) * r), a1 = round_bf16(bf16hi(v.x) * r);
    const float a2 = round_bf16(bf16lo(v.y) * r), a3 = round_bf16(bf16hi(v.y) * r);
    *(uint2*)(orow + c) = uint2{pack_bf16x2(bf16lo(wv.x) * a0, bf16hi(wv.x) * a1),
                                pack_bf16x2(bf16lo(wv.y) * a2, bf16hi(wv.y) * a3)};
  }
}

// The same for dim = 1024 * NCH (NCH <= 4): every thread keeps its NCH groups of four values in
// registers between the sum of squares and the normalization, and issues all of its loads
// (partials, residual, norm weight) before the first use.
template <int NCH>
__global__ __launch_bounds__(256) void splitk_add_rmsnorm_reg_kernel(const float* __restrict__ part, int k_split,
                                                                     int64_t rows, const uint16_t* resid_in,
                                                                     uint16_t* resid_out, const uint16_t* __restrict__ w,
                                                                     uint16_t* __restrict__ out, float eps) {
  constexpr int dim = 1024 * NCH;
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t stride = rows * dim;
  const float* pr = part + row * dim;
  float4 acc[NCH];
  uint2 rv[NCH], wv[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = tid * 4 + i * 1024;
    acc[i] = *(const float4*)(pr + c);
    rv[i] = *(const uint2*)(resid_in + row * dim + c);
    wv[i] = *(const uint2*)(w + c);
  }
  for (int s = 1; s < k_split; ++s) {  // split order, as the unfused merge sums them
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const float4 v = *(const float4*)(pr + s * stride + tid * 4 + i * 1024);
      acc[i].x += v.x; acc[i].y += v.y; acc[i].z += v.z; acc[i].w += v.w;
    }
  }
  float x[NCH][4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    x[i][0] = round_bf16(round_bf16(acc[i].x) + bf16lo(rv[i].x));
    x[i][1] = round_bf16(round_bf16(acc[i].y) + bf16hi(rv[i].x));
    x[i][2] = round_bf16(round_bf16(acc[i].z) + bf16lo(rv[i].y));
    x[i][3] = round_bf16(round_bf16(acc[i].w) + bf16hi(rv[i].y));
    ss += x[i][0] * x[i][0] + x[i][1] * x[i][1] + x[i][2] * x[i][2] + x[i][3] * x[i][3];
    *(uint2*)(resid_out + row * dim + tid * 4 + i * 1024) = uint2{pack_bf16x2(x[i][0], x[i][1]), pack_bf16x2(x[i][2], x[i][3])};
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  ss = red[0] + red[1] + red[2] + red[3];
  const float r = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const float a0 = round_bf16(x[i][0] * r), a1 = round_bf16(x[i][1] * r);
    const float a2 = round_bf16(x[i][2] * r), a3 = round_bf16(x[i][3] * r);
    *(uint2*)(out + row * dim + tid * 4 + i * 1024) =
        uint2{pack_bf16x2(bf16lo(wv[i].x) * a0, bf16hi(wv[i].x) * a1), pack_bf16x2(bf16lo(wv[i].y) * a2, bf16hi(wv[i].y) * a3)};
  }
}

// Host launchers shared with the linear entry points (pointers and shapes checked by the caller).
void launch_splitk_add_rmsnorm(const float* part, int k_split, int64_t rows, int dim, const uint16_t* resid_in,
                               uint16_t* resid_out, const uint16_t* w, uint16_t* out, float eps, hipStream_t s) {
  const dim3 grid((unsigned)rows), block(256);
  switch (dim) {
    case 1024: hipLaunchKernelGGL(splitk_add_rmsnorm_reg_kernel<1>, grid, block, 0, s, part, k_split, rows, resid_in, resid_out, w, out, eps); return;
    case 2048: hipLaunchKernelGGL(splitk_add_rmsnorm_reg_kernel<2>, grid, block, 0, s, part, k_split, rows, resid_in, resid_out, w, out, eps); return;
    case 4096: hipLaunchKernelGGL(splitk_add_rmsnorm_reg_kernel<4>, grid, block, 0, s, part, k_split, rows, resid_in, resid_out, w, out, eps); return;
    default: hipLaunchKernelGGL(splitk_add_rmsnorm_kernel, grid, block, 0, s, part, k_split, rows, dim, resid_in, resid_out, w, out, eps);
  }
}

void launch_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* w, uint16_t* out, int64_t ldo, int64_t rows, int dim,
                    float eps, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, ldx, w, out, ldo, rows, dim,
                     eps);
}

// One thread per 8-element (16-byte) piece of a (token, kv head) row of k and of v.
__global__ __launch_bounds__(256) void reshape_and_cache_kernel(const uint16_t* __restrict__ k, int64_t ldk,
                                                                const uint16_t* __restrict__ v, int64_t ldv,
                                                                int64_t tokens, int kv_heads, int dim,
                                                                const int64_t* __restrict__ slots,
                                                                uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                                int64_t num_slots) {
  const int pieces = kv_heads * dim / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= tokens * pieces) return;
  const int64_t t = idx / pieces;
  const int p = (int)(idx % pieces);
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  *(uint4*)(kc + slot * kv_heads * dim + p * 8) = *(const uint4*)(k + t * ldk + p * 8);
  *(uint4*)(vc + slot * kv_heads * dim + p * 8) = *(const uint4*)(v + t * ldv + p * 8);
}

}  // namespace msa

extern "C" int msa_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* weight, uint16_t* out, int64_t ldo,
                           int64_t rows, int64_t dim, float eps, msa_stream_t stream) {
  using namespace msa;
  if (rows == 0) return MSA_OK;
  if (!x || !weight || !out) return fail(MSA_ERR_INVALID, "msa_rmsnorm: null pointer");
  if (rows < 0 || dim <= 0 || dim > (1 << 20)) return fail(MSA_ERR_INVALID, "msa_rmsnorm: bad shape");
  if (dim % 8 != 0 || ldx % 8 != 0 || ldo % 8 != 0 || !aligned16(x) || !aligned16(out) || !aligned16(weight))
    return fail(MSA_ERR_UNSUPPORTED, "msa_rmsnorm: dim and row strides must be multiples of 8, pointers 16-byte aligned");
  if (ldx < dim || ldo < dim) return fail(MSA_ERR_INVALID, "msa_rmsnorm: row stride smaller than dim");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, x, ldx,
                     weight, out, ldo, rows, (int)dim, eps);
  return check_launch("msa_rmsnorm");
}

extern "C" int msa_add_rmsnorm(const uint16_t* residual, const uint16_t* delta, uint16_t* residual_out,
                               const uint16_t* weight, uint16_t* out, int64_t rows, int64_t dim, float eps,
                               msa_stream_t stream) {
  using namespace msa;
  if (rows == 0) return MSA_OK;
  if (!residual || !delta || !residual_out || !weight || !out) return fail(MSA_ERR_INVALID, "msa_add_rmsnorm: null pointer");
  if (rows < 0 || dim <= 0 || dim > (1 << 20)) return fail(MSA_ERR_INVALID, "msa_add_rmsnorm: bad shape");
  if (dim % 8 != 0 || !aligned16(residual) || !aligned16(delta) || !aligned16(residual_out) || !aligned16(weight) ||
      !aligned16(out))
    return fail(MSA_ERR_UNSUPPORTED, "msa_add_rmsnorm: dim must be a multiple of 8, pointers 16-byte aligned");
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                     residual, delta, residual_out, weight, out, rows, (int)dim, eps);
  return check_launch("msa_add_rmsnorm");
}

static int qk_common_checks(const char* fn, int64_t tokens, int heads, int kv_heads, int head_dim,
                            const void* q_norm_w, const void* k_norm_w, const void* cos, const void* sin,
                            const void* slot_mapping, const void* q_out, const void* k_cache, const void* v_cache) {
  using namespace msa;
  if (!q_norm_w || !k_norm_w || !cos || !sin || !slot_mapping || !q_out || !k_cache || !v_cache)
    return fail(MSA_ERR_INVALID, std::string(fn) + ": null pointer");
  if (tokens < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0)
    return fail(MSA_ERR_INVALID, std::string(fn) + ": bad head counts");
  if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 256)
    return fail(MSA_ERR_UNSUPPORTED, std::string(fn) + ": head_dim must be even and <= 256");
  return MSA_OK;
}

// The 16-byte-access kernel's preconditions (else the per-element kernel runs).
static bool qk_d128_ok(int head_dim, int64_t tokens, int heads, int kv_heads, const void* qw, const void* kw,
                       const void* cos, const void* sin, const void* q_out, const void* k_cache,
                       const void* v_cache) {
  using namespace msa;
  return head_dim == 128 && tokens * ((heads + 2 * kv_heads + 31) / 32) <= 0x7fffffff && aligned16(qw) &&
         aligned16(kw) && aligned16(cos) && aligned16(sin) && aligned16(q_out) && aligned16(k_cache) &&
         aligned16(v_cache);
}

extern "C" int msa_qk_norm_rope_cache(const uint16_t* qkv, int64_t ldqkv, int64_t tokens, int heads, int kv_heads,
                                      int head_dim, const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps,
                                      const float* cos, const float* sin, const int64_t* slot_mapping,
                                      uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, int64_t num_slots,
                                      msa_stream_t stream) {
  using namespace msa;
  if (tokens == 0) return MSA_OK;
  if (!qkv) return fail(MSA_ERR_INVALID, "msa_qk_norm_rope_cache: null pointer");
  int rc = qk_common_checks("msa_qk_norm_rope_cache", tokens, heads, kv_heads, head_dim, q_norm_w, k_norm_w, cos, sin,
                            slot_mapping, q_out, k_cache, v_cache);
  if (rc != MSA_OK) return rc;
  if (ldqkv < (int64_t)(heads + 2 * kv_heads) * head_dim)
    return fail(MSA_ERR_INVALID, "msa_qk_norm_rope_cache: ldqkv too small");
  if (qk_d128_ok(head_dim, tokens, heads, kv_heads, q_norm_w, k_norm_w, cos, sin, q_out, k_cache, v_cache) &&
      aligned16(qkv) && ldqkv % 8 == 0) {
    const int64_t blocks = tokens * ((heads + 2 * kv_heads + 31) / 32);
    hipLaunchKernelGGL(qk_norm_rope_cache_d128_kernel<false>, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, qkv, ldqkv, nullptr, 0, tokens, heads, kv_heads, q_norm_w, k_norm_w, eps,
                       cos, sin, slot_mapping, q_out, k_cache, v_cache, num_slots);
    return check_launch("msa_qk_norm_rope_cache");
  }
  const int64_t waves = tokens * (heads + 2 * kv_heads);
  hipLaunchKernelGGL(qk_norm_rope_cache_kernel<false>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, qkv, ldqkv, nullptr, 0, tokens, heads, kv_heads, head_dim, q_norm_w,
                     k_norm_w, eps, cos, sin, slot_mapping, q_out, k_cache, v_cache, num_slots);
  return check_launch("msa_qk_norm_rope_cache");
}

extern "C" int msa_qk_norm_rope_cache_splitk(const float* partials, int k_split, int64_t tokens, int heads,
                                             int kv_heads, int head_dim, const uint16_t* q_norm_w,
                                             const uint16_t* k_norm_w, float eps, const float* cos, const float* sin,
                                             const int64_t* slot_mapping, uint16_t* q_out, uint16_t* k_cache,
                                             uint16_t* v_cache, int64_t num_slots, msa_stream_t stream) {
  using namespace msa;
  if (tokens == 0) return MSA_OK;
  if (!partials || k_split < 1) return fail(MSA_ERR_INVALID, "msa_qk_norm_rope_cache_splitk: bad partials");
  int rc = qk_common_checks("msa_qk_norm_rope_cache_splitk", tokens, heads, kv_heads, head_dim, q_norm_w, k_norm_w,
                            cos, sin, slot_mapping, q_out, k_cache, v_cache);
  if (rc != MSA_OK) return rc;
  if (qk_d128_ok(head_dim, tokens, heads, kv_heads, q_norm_w, k_norm_w, cos, sin, q_out, k_cache, v_cache) &&
      aligned16(partials)) {
    const int64_t blocks = tokens * ((heads + 2 * kv_heads + 31) / 32);
    hipLaunchKernelGGL(qk_norm_rope_cache_d128_kernel<true>, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, nullptr, 0, partials, k_split, tokens, heads, kv_heads, q_norm_w,
                       k_norm_w, eps, cos, sin, slot_mapping, q_out, k_cache, v_cache, num_slots);
    return check_launch("msa_qk_norm_rope_cache_splitk");
  }
  const int64_t waves = tokens * (heads + 2 * kv_heads);
  hipLaunchKernelGGL(qk_norm_rope_cache_kernel<true>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, nullptr, 0, partials, k_split, tokens, heads, kv_heads, head_dim, q_norm_w,
                     k_norm_w, eps, cos, sin, slot_mapping, q_out, k_cache, v_cache, num_slots);
  return check_launch("msa_qk_norm_rope_cache_splitk");
}

extern "C" int msa_splitk_add_rmsnorm(const float* partials, int k_split, const uint16_t* residual,
                                      uint16_t* residual_out, const uint16_t* weight, uint16_t* out, int64_t rows,
                                      int64_t dim, float eps, msa_stream_t stream) {
  using namespace msa;
  if (rows == 0) return MSA_OK;
  if (!partials || !residual || !residual_out || !weight || !out)
    return fail(MSA_ERR_INVALID, "msa_splitk_add_rmsnorm: null pointer");
  if (k_split < 1 || rows < 0 || dim <= 0 || dim > (1 << 20) || rows > 0x7fffffff)
    return fail(MSA_ERR_INVALID, "msa_splitk_add_rmsnorm: bad shape");
  if (dim % 4 != 0 || !aligned16(partials) || (reinterpret_cast<uintptr_t>(residual) & 7u) ||
      (reinterpret_cast<uintptr_t>(residual_out) & 7u) || (reinterpret_cast<uintptr_t>(weight) & 7u) ||
      (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(MSA_ERR_UNSUPPORTED, "msa_splitk_add_rmsnorm: dim must be a multiple of 4, pointers aligned");
  launch_splitk_add_rmsnorm(partials, k_split, rows, (int)dim, residual, residual_out, weight, out, eps,
                            (hipStream_t)stream);
  return check_launch("msa_splitk_add_rmsnorm");
}

extern "C" int msa_reshape_and_cache(const uint16_t* k, int64_t ldk, const uint16_t* v, int64_t ldv, int64_t tokens,
                                     int kv_heads, int head_dim, const int64_t* slot_mapping, uint16_t* k_cache,
                                     uint16_t* v_cache, int64_t num_slots, msa_stream_t stream) {
  using namespace msa;
  if (tokens == 0) return MSA_OK;
  if (!k || !v || !slot_mapping || !k_cache || !v_cache) return fail(MSA_ERR_INVALID, "msa_reshape_and_cache: null pointer");
  if (tokens < 0 || kv_heads <= 0 || head_dim <= 0) return fail(MSA_ERR_INVALID, "msa_reshape_and_cache: bad shape");
  if ((kv_heads * head_dim) % 8 != 0 || ldk % 8 != 0 || ldv % 8 != 0 || !aligned16(k) || !aligned16(v) ||
      !aligned16(k_cache) || !aligned16(v_cache))
    return fail(MSA_ERR_UNSUPPORTED, "msa_reshape_and_cache: rows must be 16-byte aligned multiples of 8 elements");
  if (ldk < (int64_t)kv_heads * head_dim || ldv < (int64_t)kv_heads * head_dim)
    return fail(MSA_ERR_INVALID, "msa_reshape_and_cache: row stride too small");
  const int64_t threads = tokens * (kv_heads * head_dim / 8);
  hipLaunchKernelGGL(reshape_and_cache_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, k, ldk, v, ldv, tokens, kv_heads, head_dim, slot_mapping, k_cache, v_cache,
                     num_slots);
  return check_launch("msa_reshape_and_cache");
}
