// The reference's unfused GPU sequence for a dense layer, on this library's
// kernels, for comparison with the fused launch.
//
// The reference's GPU pipeline lowers relu(X @ W + b) to three kernels run
// one after another: linalg.fill of the output with zeros, the matmul, and
// the merged bias + ReLU generic as a separate elementwise pass over the
// output (reference cpp/src/MLIRLowering.cpp:495-518; three launches per call,
// tests/gpu/test_gpu_execution.py:149-154). The same sequence here is: a fill
// kernel, the tiled / small-M GEMM with no epilogue, and the elementwise
// bias + activation kernel below. Its results equal the fused launch's bit
// for bit: the epilogue applies the same fp32 operations to the same fp32
// accumulator values, only after a round trip through memory.
#include "common.hpp"
#include "kernels.hpp"

namespace edsl {
namespace {

// Y[M][N] = 0 (linalg.fill). Four columns per thread when the rows allow
// 16-byte stores.
__global__ void __launch_bounds__(256) fill_zero_f32_kernel(float* Y, int64_t ldy, int M, int N, int vec) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (vec) {
    const int n4 = N / 4;
    if (i >= (int64_t)M * n4) return;
    const int64_t r = i / n4, c = 4 * (i % n4);
    *reinterpret_cast<f32x4*>(Y + r * ldy + c) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  } else {
    if (i >= (int64_t)M * N) return;
    Y[(i / N) * ldy + i % N] = 0.0f;
  }
}

// Y[m][n] = act(Y[m][n] + bias[n]) in place: the bias / activation generic.
template <int EPI>
__global__ void __launch_bounds__(256) bias_act_f32_kernel(float* Y, int64_t ldy, const float* bias, int M, int N,
                                                           float alpha, int vec) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (vec) {
    const int n4 = N / 4;
    if (i >= (int64_t)M * n4) return;
    const int64_t r = i / n4, c = 4 * (i % n4);
    f32x4 y = *reinterpret_cast<const f32x4*>(Y + r * ldy + c);
    f32x4 b = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (epi_has_bias(EPI)) b = *reinterpret_cast<const f32x4*>(bias + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = apply_epilogue_f32<EPI>(y[e], b[e], alpha);
    *reinterpret_cast<f32x4*>(Y + r * ldy + c) = y;
  } else {
    if (i >= (int64_t)M * N) return;
    const int64_t r = i / N, c = i % N;
    const float b = epi_has_bias(EPI) ? bias[c] : 0.0f;
    Y[r * ldy + c] = apply_epilogue_f32<EPI>(Y[r * ldy + c], b, alpha);
  }
}

}  // namespace

hipError_t launch_fill_zero_f32(float* Y, int64_t ldy, int M, int N, hipStream_t stream) {
  if (M <= 0 || N <= 0) return hipSuccess;
  const int vec = (reinterpret_cast<uintptr_t>(Y) % 16 == 0) && ldy % 4 == 0 && N % 4 == 0;
  const int64_t items = vec ? (int64_t)M * (N / 4) : (int64_t)M * N;
  hipLaunchKernelGGL(fill_zero_f32_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, stream, Y, ldy, M,
                     N, vec);
  return hipGetLastError();
}

hipError_t launch_bias_act_f32(float* Y, int64_t ldy, const float* bias, int M, int N, int epi, float alpha,
                               hipStream_t stream) {
  if (M <= 0 || N <= 0 || epi == epi_code(false, ACT_NONE)) return hipSuccess;
  const int vec = (reinterpret_cast<uintptr_t>(Y) % 16 == 0) && ldy % 4 == 0 && N % 4 == 0 &&
                  (!epi_has_bias(epi) || reinterpret_cast<uintptr_t>(bias) % 16 == 0);
  const int64_t items = vec ? (int64_t)M * (N / 4) : (int64_t)M * N;
  const dim3 grid((unsigned)((items + 255) / 256)), block(256);
  switch (epi) {
    case epi_code(true, ACT_NONE):
      hipLaunchKernelGGL(bias_act_f32_kernel<epi_code(true, ACT_NONE)>, grid, block, 0, stream, Y, ldy, bias, M, N,
                         alpha, vec);
      break;
    case epi_code(false, ACT_RELU):
      hipLaunchKernelGGL(bias_act_f32_kernel<epi_code(false, ACT_RELU)>, grid, block, 0, stream, Y, ldy, bias, M, N,
                         alpha, vec);
      break;
    case epi_code(true, ACT_RELU):
      hipLaunchKernelGGL(bias_act_f32_kernel<epi_code(true, ACT_RELU)>, grid, block, 0, stream, Y, ldy, bias, M, N,
                         alpha, vec);
      break;
    case epi_code(false, ACT_LEAKY):
      hipLaunchKernelGGL(bias_act_f32_kernel<epi_code(false, ACT_LEAKY)>, grid, block, 0, stream, Y, ldy, bias, M,
                         N, alpha, vec);
      break;
    case epi_code(true, ACT_LEAKY):
      hipLaunchKernelGGL(bias_act_f32_kernel<epi_code(true, ACT_LEAKY)>, grid, block, 0, stream, Y, ldy, bias, M,
                         N, alpha, vec);
      break;
    case epi_code(false, ACT_IF_RELU):
      hipLaunchKernelGGL(bias_act_f32_kernel<epi_code(false, ACT_IF_RELU)>, grid, block, 0, stream, Y, ldy, bias, M,
                         N, alpha, vec);
      break;
    case epi_code(true, ACT_IF_RELU):
      hipLaunchKernelGGL(bias_act_f32_kernel<epi_code(true, ACT_IF_RELU)>, grid, block, 0, stream, Y, ldy, bias, M,
                         N, alpha, vec);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace edsl
