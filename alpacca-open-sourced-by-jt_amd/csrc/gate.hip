// Sigmoid output gate (out = values * sigmoid(gate)) and SiLU
// (out = x * sigmoid(x)), elementwise.
#include "alpx_common.h"

namespace alpx {
namespace {

template <typename T, typename TO>
__global__ void __launch_bounds__(256)
sigmoid_gate_kernel(const T* __restrict__ values, const T* __restrict__ gate, TO* out,
                    int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = from_f32<TO>(to_f32(values[i]) * stable_sigmoid(to_f32(gate[i])));
}

// gate == nullptr: SiLU of values.
template <typename T, typename TO>
__global__ void __launch_bounds__(256)
silu_kernel(const T* __restrict__ values, TO* out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float x = to_f32(values[i]);
    out[i] = from_f32<TO>(x * stable_sigmoid(x));
  }
}

template <typename T>
int launch(const void* v, const void* g, void* out, int64_t n, int out_dtype, hipStream_t s) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  dim3 grid((unsigned)blocks);
  if (!g) {
    switch (out_dtype) {
      case ALPX_F32:
        hipLaunchKernelGGL((silu_kernel<T, float>), grid, dim3(256), 0, s, (const T*)v, (float*)out, n);
        break;
      case ALPX_F16:
        hipLaunchKernelGGL((silu_kernel<T, f16_t>), grid, dim3(256), 0, s, (const T*)v, (f16_t*)out, n);
        break;
      default:
        hipLaunchKernelGGL((silu_kernel<T, bf16_t>), grid, dim3(256), 0, s, (const T*)v, (bf16_t*)out, n);
        break;
    }
    return check_launch("alpx_silu");
  }
  switch (out_dtype) {
    case ALPX_F32:
      hipLaunchKernelGGL((sigmoid_gate_kernel<T, float>), grid, dim3(256), 0, s, (const T*)v,
                         (const T*)g, (float*)out, n);
      break;
    case ALPX_F16:
      hipLaunchKernelGGL((sigmoid_gate_kernel<T, f16_t>), grid, dim3(256), 0, s, (const T*)v,
                         (const T*)g, (f16_t*)out, n);
      break;
    default:
      hipLaunchKernelGGL((sigmoid_gate_kernel<T, bf16_t>), grid, dim3(256), 0, s, (const T*)v,
                         (const T*)g, (bf16_t*)out, n);
      break;
  }
  return check_launch("alpx_sigmoid_gate");
}

}  // namespace
}  // namespace alpx

extern "C" int alpx_sigmoid_gate(const void* values, const void* gate, void* out, int64_t n,
                                 int dtype, int out_dtype, void* stream) {
  using namespace alpx;
  if (!values || !gate || !out) return fail(ALPX_EINVAL, "alpx_sigmoid_gate: null buffer");
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype))
    return fail(ALPX_EINVAL, "alpx_sigmoid_gate: unknown dtype");
  if (n < 0) return fail(ALPX_EINVAL, "alpx_sigmoid_gate: negative size");
  if (n == 0) return ALPX_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ALPX_F32: return launch<float>(values, gate, out, n, out_dtype, s);
    case ALPX_F16: return launch<f16_t>(values, gate, out, n, out_dtype, s);
    default: return launch<bf16_t>(values, gate, out, n, out_dtype, s);
  }
}

extern "C" int alpx_silu(const void* values, void* out, int64_t n, int dtype, int out_dtype,
                         void* stream) {
  using namespace alpx;
  if (!values || !out) return fail(ALPX_EINVAL, "alpx_silu: null buffer");
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return fail(ALPX_EINVAL, "alpx_silu: unknown dtype");
  if (n < 0) return fail(ALPX_EINVAL, "alpx_silu: negative size");
  if (n == 0) return ALPX_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case ALPX_F32: return launch<float>(values, nullptr, out, n, out_dtype, s);
    case ALPX_F16: return launch<f16_t>(values, nullptr, out, n, out_dtype, s);
    default: return launch<bf16_t>(values, nullptr, out, n, out_dtype, s);
  }
}
