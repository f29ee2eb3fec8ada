// Element-wise and layout kernels of the MoE FFN path.
//
//   swiglu   gate * silu(up)  (components/activation/swiglu.mlir:37-47,
//            oracles/activation.py:11-21)
//   combine  out[t, :] = sum_{s=0..k-1} y[s*T + t, :] in slot order: the
//            routing-weight product is applied by the down GEMM's epilogue,
//            this is the slot reduction + transpose of
//            moe_ffn_block.mlir:179-206 (oracles/moe.py:126-132)
//   transpose / zero rows / fill: layout plumbing of the standalone
//            mul_mat_id, whose input and output are feature-major
//            [n, k, T] (mul_mat_id.mlir:63-117).
#include "common.h"
#include "launch.h"

namespace fmoe {
namespace {

constexpr int kThreads = 256;

template <typename T>
__device__ __forceinline__ float ldf(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ldf<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ldf<bf16_t>(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }

template <typename T>
__device__ __forceinline__ void stf(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void stf<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void stf<bf16_t>(bf16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

template <typename T>
__global__ __launch_bounds__(kThreads) void swiglu_kernel(const T* __restrict__ gate,
                                                          const T* __restrict__ up,
                                                          T* __restrict__ out, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const float g = ldf(gate, i);
    const float u = ldf(up, i);
    stf(out, i, g * (u / (1.f + expf(-u))));
  }
}

// out[t, c] = sum_s (y_0 + y_1 + ...)[s*T + t, c]: slots in order, K-split
// partials summed first in split order.
template <typename TY, typename TO>
__global__ __launch_bounds__(kThreads) void combine_kernel(const TY* __restrict__ y,
                                                           TO* __restrict__ out, int n_tokens,
                                                           int k, int n_embd, int nsplit,
                                                           int64_t split_stride) {
  const int64_t total = static_cast<int64_t>(n_tokens) * n_embd;
  const int64_t slot_stride = total;  // y rows s*T + t -> element offset s*T*H + t*H
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    float acc = 0.f;
    for (int s = 0; s < k; ++s) {
      float v = ldf(y, i + s * slot_stride);
      for (int p = 1; p < nsplit; ++p) v += ldf(y, i + s * slot_stride + p * split_stride);
      acc = s == 0 ? v : acc + v;
    }
    stf(out, i, acc);
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void transpose_kernel(const T* __restrict__ in,
                                                             T* __restrict__ out, int64_t rows,
                                                             int64_t cols) {
  __shared__ T tile[32][33];
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int tx = threadIdx.x & 31;
  const int ty = threadIdx.x >> 5;  // 0..7
  for (int j = ty; j < 32; j += 8) {
    const int64_t r = r0 + j, c = c0 + tx;
    if (r < rows && c < cols) tile[j][tx] = in[r * cols + c];
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    const int64_t c = c0 + j, r = r0 + tx;
    if (r < rows && c < cols) out[c * rows + r] = tile[tx][j];
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void zero_invalid_rows_kernel(const int* __restrict__ ids,
                                                                     int n_assign, int n_expert,
                                                                     T* __restrict__ y,
                                                                     int64_t width) {
  const int f = blockIdx.x;
  if (f >= n_assign) return;
  const int e = ids[f];
  if (e >= 0 && e < n_expert) return;
  for (int64_t c = threadIdx.x; c < width; c += kThreads) y[f * width + c] = T(0);
}

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(uint32_t* __restrict__ p, size_t n) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * kThreads)
    p[i] = 0u;
}

unsigned grid_for(int64_t n) {
  int64_t b = (n + kThreads - 1) / kThreads;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return static_cast<unsigned>(b);
}

}  // namespace

hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype,
                         hipStream_t stream) {
  if (n == 0) return hipSuccess;
  if (dtype == DT_F32)
    hipLaunchKernelGGL(swiglu_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, stream,
                       static_cast<const float*>(gate), static_cast<const float*>(up),
                       static_cast<float*>(out), n);
  else
    hipLaunchKernelGGL(swiglu_kernel<bf16_t>, dim3(grid_for(n)), dim3(kThreads), 0, stream,
                       static_cast<const bf16_t*>(gate), static_cast<const bf16_t*>(up),
                       static_cast<bf16_t*>(out), n);
  return hipGetLastError();
}

hipError_t launch_combine(const void* y, int y_dtype, void* out, int out_dtype, int n_tokens,
                          int k, int n_embd, int nsplit, int64_t split_stride, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(n_tokens) * n_embd;
  if (total == 0) return hipSuccess;
  const dim3 grid(grid_for(total));
  if (y_dtype == DT_F32 && out_dtype == DT_F32)
    hipLaunchKernelGGL((combine_kernel<float, float>), grid, dim3(kThreads), 0, stream,
                       static_cast<const float*>(y), static_cast<float*>(out), n_tokens, k, n_embd, nsplit,
                       split_stride);
  else if (y_dtype == DT_F32)
    hipLaunchKernelGGL((combine_kernel<float, bf16_t>), grid, dim3(kThreads), 0, stream,
                       static_cast<const float*>(y), static_cast<bf16_t*>(out), n_tokens, k, n_embd, nsplit,
                       split_stride);
  else if (out_dtype == DT_F32)
    hipLaunchKernelGGL((combine_kernel<bf16_t, float>), grid, dim3(kThreads), 0, stream,
                       static_cast<const bf16_t*>(y), static_cast<float*>(out), n_tokens, k, n_embd, nsplit,
                       split_stride);
  else
    hipLaunchKernelGGL((combine_kernel<bf16_t, bf16_t>), grid, dim3(kThreads), 0, stream,
                       static_cast<const bf16_t*>(y), static_cast<bf16_t*>(out), n_tokens, k, n_embd, nsplit,
                       split_stride);
  return hipGetLastError();
}

hipError_t launch_transpose(const void* in, void* out, int64_t rows, int64_t cols, int dtype,
                            hipStream_t stream) {
  if (rows == 0 || cols == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((cols + 31) / 32), static_cast<unsigned>((rows + 31) / 32));
  if (grid.y > 65535) return hipErrorInvalidValue;
  if (dtype == DT_F32)
    hipLaunchKernelGGL(transpose_kernel<float>, grid, dim3(kThreads), 0, stream,
                       static_cast<const float*>(in), static_cast<float*>(out), rows, cols);
  else
    hipLaunchKernelGGL(transpose_kernel<bf16_t>, grid, dim3(kThreads), 0, stream,
                       static_cast<const bf16_t*>(in), static_cast<bf16_t*>(out), rows, cols);
  return hipGetLastError();
}

hipError_t launch_zero_invalid_rows(const int* ids, int n_assign, int n_expert, void* y, int dtype,
                                    int64_t width, hipStream_t stream) {
  if (n_assign == 0 || width == 0) return hipSuccess;
  if (dtype == DT_F32)
    hipLaunchKernelGGL(zero_invalid_rows_kernel<float>, dim3(n_assign), dim3(kThreads), 0, stream,
                       ids, n_assign, n_expert, static_cast<float*>(y), width);
  else
    hipLaunchKernelGGL(zero_invalid_rows_kernel<bf16_t>, dim3(n_assign), dim3(kThreads), 0, stream,
                       ids, n_assign, n_expert, static_cast<bf16_t*>(y), width);
  return hipGetLastError();
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream) {
  const size_t n = bytes / 4;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(static_cast<int64_t>(n))), dim3(kThreads), 0,
                     stream, static_cast<uint32_t*>(p), n);
  return hipGetLastError();
}

}  // namespace fmoe
