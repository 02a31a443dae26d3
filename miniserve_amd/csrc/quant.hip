// Per-row symmetric int8 quantization of a weight matrix (the pack step of the int8 linears).
//
// One workgroup per row: a max-abs reduction, then scale32 = max(amax, 1e-8) / 127 with IEEE
// division (hipcc divides float32 correctly rounded by default), q = rint(w / scale32) -- rint
// rounds half to even like torch.round -- clamped to [-127, 127], and the scale stored as bf16
// with round-to-nearest-even. This reproduces quant/int8.py:27-32 bit for bit.
#include "common.h"

namespace msa {

template <typename T>
__device__ __forceinline__ float load_w(const T* p);
template <>
__device__ __forceinline__ float load_w<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }
template <>
__device__ __forceinline__ float load_w<float>(const float* p) { return *p; }

template <typename T>
__global__ __launch_bounds__(256) void int8_quantize_kernel(const T* __restrict__ w, int64_t cols,
                                                            int8_t* __restrict__ q,
                                                            uint16_t* __restrict__ scale) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const T* wr = w + row * cols;
  float amax = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) amax = fmaxf(amax, fabsf(load_w(wr + c)));
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fmaxf(amax, 1e-8f) / 127.0f;
  int8_t* qr = q + row * cols;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    float v = rintf(load_w(wr + c) / s);
    v = fminf(fmaxf(v, -127.f), 127.f);
    qr[c] = (int8_t)(int)v;
  }
  if (threadIdx.x == 0) scale[row] = f32_to_bf16(s);
}

}  // namespace msa

extern "C" int msa_int8_quantize(const void* weight, int weight_dtype, int64_t rows, int64_t cols,
                                 int8_t* qweight, uint16_t* scale, msa_stream_t stream) {
  using namespace msa;
  if (!weight || !qweight || !scale) return fail(MSA_ERR_INVALID, "msa_int8_quantize: null pointer");
  if (rows <= 0 || cols <= 0 || rows > 0x7fffffff)
    return fail(MSA_ERR_INVALID, "msa_int8_quantize: rows and cols must be positive");
  hipStream_t s = (hipStream_t)stream;
  if (weight_dtype == 0) {
    hipLaunchKernelGGL(int8_quantize_kernel<uint16_t>, dim3((unsigned)rows), dim3(256), 0, s,
                       (const uint16_t*)weight, cols, qweight, scale);
  } else if (weight_dtype == 1) {
    hipLaunchKernelGGL(int8_quantize_kernel<float>, dim3((unsigned)rows), dim3(256), 0, s,
                       (const float*)weight, cols, qweight, scale);
  } else {
    return fail(MSA_ERR_UNSUPPORTED, "msa_int8_quantize: weight_dtype must be 0 (bf16) or 1 (float32)");
  }
  return check_launch("msa_int8_quantize");
}
