// One-time expert-weight packing: reference layout [n_out, n_in, E] (expert
// innermost, components/moe/moe_ffn_block.mlir:37-39) -> per-expert operand
// layout (packed_format / packed_offset in launch.h: MFMA-ready 1 KiB blocks
// when the shape allows, else [E][n_out][n_in] row-major).  The reference instead transposes every weight on
// every call (components/moe/mul_mat_id.mlir:37-48).
//
// fp8 (OCP e4m3fn) packing quantises each output channel (o, e):
//   scale = max_i |w[o, i, e]| / 448 (1 for an all-zero channel)
//   code  = RNE(w / scale), saturating at +-448.
// Scales are written [E][n_out].
#include "common.h"
#include "launch.h"

namespace fmoe {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxExpert = 1024;

__device__ __forceinline__ float load_src(const void* src, int dt, int64_t i) {
  if (dt == DT_F32) return static_cast<const float*>(src)[i];
  if (dt == DT_BF16) return bf16_to_f32(static_cast<const bf16_t*>(src)[i]);
  return e4m3fn_to_f32(static_cast<const f8_t*>(src)[i]);
}

// One block per output row o.  Reads the contiguous [n_in, E] slab of row o
// and writes E rows of n_in elements.
__global__ __launch_bounds__(kThreads) void pack_kernel(const void* __restrict__ src, int src_dt,
                                                        const float* __restrict__ src_scales,
                                                        int n_out, int n_in, int n_expert,
                                                        int dst_dt, void* __restrict__ dst,
                                                        float* __restrict__ dst_scales) {
  __shared__ uint32_t amax_bits[kMaxExpert];
  __shared__ float scale[kMaxExpert];
  const int o = blockIdx.x;
  const int fmt = packed_format(n_out, n_in, dst_dt);
  const int64_t slab = static_cast<int64_t>(n_in) * n_expert;
  const int64_t src0 = static_cast<int64_t>(o) * slab;

  if (dst_dt == DT_F8 && src_dt != DT_F8) {
    for (int e = threadIdx.x; e < n_expert; e += kThreads) amax_bits[e] = 0;
    __syncthreads();
    for (int64_t idx = threadIdx.x; idx < slab; idx += kThreads) {
      const int e = static_cast<int>(idx % n_expert);
      const float v = fabsf(load_src(src, src_dt, src0 + idx));
      atomicMax(&amax_bits[e], __float_as_uint(v));  // non-negative floats order as uints
    }
    __syncthreads();
    for (int e = threadIdx.x; e < n_expert; e += kThreads) {
      const float amax = __uint_as_float(amax_bits[e]);
      const float s = amax > 0.f ? amax / 448.0f : 1.0f;
      scale[e] = s;
      dst_scales[static_cast<int64_t>(e) * n_out + o] = s;
    }
    __syncthreads();
  } else if (dst_dt == DT_F8) {
    // Already quantised: copy codes, transpose scales [n_out][E] -> [E][n_out].
    for (int e = threadIdx.x; e < n_expert; e += kThreads)
      dst_scales[static_cast<int64_t>(e) * n_out + o] = src_scales[static_cast<int64_t>(o) * n_expert + e];
  }

  for (int64_t idx = threadIdx.x; idx < slab; idx += kThreads) {
    const int e = static_cast<int>(idx % n_expert);
    const int64_t i = idx / n_expert;
    const int64_t d = packed_offset(fmt, dst_dt, e, o, i, n_out, n_in);
    if (dst_dt == DT_F8) {
      if (src_dt == DT_F8) {
        static_cast<f8_t*>(dst)[d] = static_cast<const f8_t*>(src)[src0 + idx];
      } else {
        const float v = load_src(src, src_dt, src0 + idx);
        static_cast<f8_t*>(dst)[d] = static_cast<f8_t>(f32_to_e4m3fn(v / scale[e]));
      }
    } else {
      const float v = load_src(src, src_dt, src0 + idx);
      if (dst_dt == DT_F32)
        static_cast<float*>(dst)[d] = v;
      else
        static_cast<bf16_t*>(dst)[d] = f32_to_bf16(v);
    }
  }
}

// Dense linear weight src [n_in, n_part] row-major (the reference's
// `x @ W` operand, attention_block_decode.mlir:104-118) -> rows
// [row0, row0 + n_part) of a one-expert packed [n_total, n_in] weight.  One
// block per output row: a strided column read (one-time packing).
__global__ __launch_bounds__(kThreads) void pack_linear_kernel(const void* __restrict__ src, int src_dt, int n_in,
                                                               int n_part, int row0, int n_total, int dst_dt,
                                                               void* __restrict__ dst, float* __restrict__ dst_scales) {
  __shared__ float red[kThreads / kWave];
  const int o = blockIdx.x;
  const int og = row0 + o;
  const int fmt = packed_format(n_total, n_in, dst_dt);
  float scale = 1.f;
  if (dst_dt == DT_F8) {
    float m = 0.f;
    for (int i = threadIdx.x; i < n_in; i += kThreads)
      m = fmaxf(m, fabsf(load_src(src, src_dt, static_cast<int64_t>(i) * n_part + o)));
    m = wave_max(m);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < kThreads / kWave; ++w) m = fmaxf(m, red[w]);
    scale = m > 0.f ? m / 448.0f : 1.0f;
    if (threadIdx.x == 0) dst_scales[og] = scale;
  }
  for (int i = threadIdx.x; i < n_in; i += kThreads) {
    const float v = load_src(src, src_dt, static_cast<int64_t>(i) * n_part + o);
    const int64_t d = packed_offset(fmt, dst_dt, 0, og, i, n_total, n_in);
    if (dst_dt == DT_F8)
      static_cast<f8_t*>(dst)[d] = static_cast<f8_t>(f32_to_e4m3fn(v / scale));
    else if (dst_dt == DT_F32)
      static_cast<float*>(dst)[d] = v;
    else
      static_cast<bf16_t*>(dst)[d] = f32_to_bf16(v);
  }
}

}  // namespace

hipError_t launch_pack_linear(const void* src, int src_dtype, int n_in, int n_part, int row0, int n_total,
                              int dst_dtype, void* dst, float* dst_scales, hipStream_t stream) {
  if (n_part == 0 || n_in == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_linear_kernel, dim3(n_part), dim3(kThreads), 0, stream, src, src_dtype, n_in, n_part, row0,
                     n_total, dst_dtype, dst, dst_scales);
  return hipGetLastError();
}

hipError_t launch_pack(const void* src, int src_dtype, const float* src_scales, int n_out,
                       int n_in, int n_expert, int dst_dtype, void* dst, float* dst_scales,
                       hipStream_t stream) {
  if (n_expert > kMaxExpert) return hipErrorInvalidValue;
  if (n_out == 0 || n_in == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_kernel, dim3(n_out), dim3(kThreads), 0, stream, src, src_dtype,
                     src_scales, n_out, n_in, n_expert, dst_dtype, dst, dst_scales);
  return hipGetLastError();
}

}  // namespace fmoe
