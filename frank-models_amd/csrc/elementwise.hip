// Element-wise and layout kernels of the MoE FFN path.
//
//   swiglu   gate * silu(up)  (components/activation/swiglu.mlir:37-47,
//            oracles/activation.py:11-21)
//   combine  out[t, :] = sum_{s=0..k-1} y[s*T + t, :] in slot order: the
//            routing-weight product is applied by the down GEMM's epilogue,
//            this is the slot reduction + transpose of
//            moe_ffn_block.mlir:179-206 (oracles/moe.py:126-132); optionally
//            plus the layer's residual, residual + moe_out
//            (transformer_layer_moe_prefill.mlir:229-242)
//   rms_norm (x / sqrt(mean(x^2) + eps)) * weight per row
//            (components/normalization/rms_norm.mlir:18-85,
//            oracles/normalization.py:10-43)
//   transpose / zero rows / fill: layout plumbing of the standalone
//            mul_mat_id, whose input and output are feature-major
//            [n, k, T] (mul_mat_id.mlir:63-117).
#include "common.h"
#include "launch.h"

#include <algorithm>

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

// V consecutive elements (V = 4 or 8: 16-byte fp32 loads, 8- or 16-byte
// bf16 loads).
template <int V>
__device__ __forceinline__ void ldv(const float* p, int64_t i, float* v) {
  if constexpr (V % 4 == 0) {
#pragma unroll
    for (int c = 0; c < V / 4; ++c) {
      const f32x4_t q = *reinterpret_cast<const f32x4_t*>(p + i + 4 * c);
      v[4 * c] = q[0], v[4 * c + 1] = q[1], v[4 * c + 2] = q[2], v[4 * c + 3] = q[3];
    }
  } else {
    v[0] = p[i];
  }
}
__device__ __forceinline__ void unpack_bf16x2(uint32_t q, float* v) {
  v[0] = __uint_as_float(q << 16), v[1] = __uint_as_float(q & 0xFFFF0000u);
}
template <int V>
__device__ __forceinline__ void ldv(const bf16_t* p, int64_t i, float* v) {
  if constexpr (V == 8) {
    const u32x4_t q = *reinterpret_cast<const u32x4_t*>(p + i);
#pragma unroll
    for (int c = 0; c < 4; ++c) unpack_bf16x2(q[c], v + 2 * c);
  } else if constexpr (V == 4) {
    const u32x2_t q = *reinterpret_cast<const u32x2_t*>(p + i);
    unpack_bf16x2(q[0], v), unpack_bf16x2(q[1], v + 2);
  } else {
    v[0] = bf16_to_f32(p[i]);
  }
}
template <int V>
__device__ __forceinline__ void stv(float* p, int64_t i, const float* v) {
  if constexpr (V % 4 == 0) {
#pragma unroll
    for (int c = 0; c < V / 4; ++c)
      *reinterpret_cast<f32x4_t*>(p + i + 4 * c) = f32x4_t{v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]};
  } else {
    p[i] = v[0];
  }
}
template <int V>
__device__ __forceinline__ void stv(bf16_t* p, int64_t i, const float* v) {
  if constexpr (V == 8)
    *reinterpret_cast<u32x4_t*>(p + i) = u32x4_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                 pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
  else if constexpr (V == 4)
    *reinterpret_cast<u32x2_t*>(p + i) = u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  else
    p[i] = f32_to_bf16(v[0]);
}

// out[t, c] = [residual[t, c] +] sum_s (y_0 + y_1 + ...)[s*T + t, c]: K-split
// partials summed first in split order, then slots in order, in fp32; one
// rounding to the output type.
// out may alias residual: each element is read and then written by one thread.
template <typename TY, typename TO, int V>
__global__ __launch_bounds__(kThreads) void combine_kernel(const TY* __restrict__ y,
                                                           const TO* residual,
                                                           TO* out, int n_tokens,
                                                           int k, int n_embd, int nsplit,
                                                           int64_t split_stride) {
  const int64_t total = static_cast<int64_t>(n_tokens) * n_embd;
  const int64_t slot_stride = total;  // y rows s*T + t -> element offset s*T*H + t*H
  for (int64_t i = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * V; i < total;
       i += static_cast<int64_t>(gridDim.x) * kThreads * V) {
    float acc[V], v[V], p[V];
    for (int s = 0; s < k; ++s) {
      ldv<V>(y, i + s * slot_stride, v);
      for (int q = 1; q < nsplit; ++q) {
        ldv<V>(y, i + s * slot_stride + q * split_stride, p);
#pragma unroll
        for (int j = 0; j < V; ++j) v[j] += p[j];
      }
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] = s == 0 ? v[j] : acc[j] + v[j];
    }
    if (residual) {
      ldv<V>(residual, i, p);
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] = p[j] + acc[j];
    }
    stv<V>(out, i, acc);
  }
}

// dst row p = src row order[p] % n_tokens, written K-blocked (kb_offset):
// each thread copies one 16-byte chunk.  A wave takes 16 rows x 64 bytes of
// one 32-column block, so its stores are one contiguous 1 KiB run; the
// waves of a row group walk its blocks in order, so the source rows are read
// in whole cache lines by neighbouring waves.
__global__ __launch_bounds__(kThreads) void gather_rows_kb_kernel(const bf16_t* __restrict__ src,
                                                                  const int* __restrict__ order, int n_rows,
                                                                  int n_tokens, int n_cols,
                                                                  bf16_t* __restrict__ dst) {
  const int64_t nblk = n_cols / 32;
  const int64_t total = (static_cast<int64_t>(n_rows) + 15) / 16 * nblk * kWave;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int lane = static_cast<int>(i & (kWave - 1));
    const int64_t w = i / kWave;
    const int64_t rg = w / nblk, j = w - rg * nblk;
    const int64_t p = rg * 16 + (lane >> 2);
    if (p >= n_rows) continue;
    const int ch = lane & 3;
    const int64_t srow = static_cast<uint32_t>(order[p]) % static_cast<uint32_t>(n_tokens);
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(src + srow * n_cols + j * 32 + ch * 8);
    *reinterpret_cast<u32x4_t*>(dst + (j * n_rows + p) * 32 + ch * 8) = v;
  }
}

// max|row| of src [n_rows, n_cols] bf16 as float bits, one wave per row
// (16-byte loads, four in flight per lane); the first n_zero words of
// zero_out (may be null) are cleared on the way.
__global__ __launch_bounds__(kThreads) void row_absmax_kernel(const bf16_t* __restrict__ src, int n_rows, int n_cols,
                                                              unsigned* __restrict__ amax_out,
                                                              unsigned* __restrict__ zero_out, int n_zero) {
  const int lane = threadIdx.x & (kWave - 1);
  const int waves = kThreads / kWave;
  if (zero_out)
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n_zero;
         i += static_cast<int64_t>(gridDim.x) * kThreads)
      zero_out[i] = 0u;
  const int n_chunks = n_cols / 8;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * waves + threadIdx.x / kWave; r < n_rows;
       r += static_cast<int64_t>(gridDim.x) * waves) {
    const u32x4_t* row = reinterpret_cast<const u32x4_t*>(src + r * n_cols);
    float m = 0.f;
    for (int c = lane; c < n_chunks; c += 4 * kWave) {
      u32x4_t v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (c + u * kWave < n_chunks) v[u] = row[c + u * kWave];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (c + u * kWave < n_chunks) m = fmaxf(m, absmax_bf16x8(v[u]));
    }
    m = wave_max(m);
    if (lane == 0) amax_out[r] = __float_as_uint(m);
  }
}

// A block of 256 threads quantises pieces 32 y .. 32 y + 31 of rows
// p0 .. p0+15 (p0 = 16 x).  row_amax, when given, holds max|v| of each
// source row (indexed like src); otherwise each wave first reduces max|v|
// of four rows (coalesced 16-byte loads) into LDS.  Then wave w
// writes pieces j = 32 y + w + 4 t (t < 8, all loads first): lane
// (r = lane / 4, g = lane % 4) converts row p0+r's inputs 64j + 8g + [0, 8)
// and 64j + 32 + 8g + [0, 8) (the packed fp8 weights' lane order) and stores
// them as chunk g of the piece, so each store instruction writes the 16
// rows' pieces as one contiguous 1 KiB run.
__global__ __launch_bounds__(kThreads) void quantize_rows_kb_kernel(const bf16_t* __restrict__ src,
                                                                    const int* __restrict__ order, int n_rows,
                                                                    int n_tokens, int n_cols,
                                                                    const unsigned* __restrict__ row_amax,
                                                                    uint8_t* __restrict__ dst_q,
                                                                    float* __restrict__ dst_scale,
                                                                    unsigned* __restrict__ zero_out,
                                                                    uint8_t* __restrict__ dst_lo) {
  __shared__ int64_t s_row[16];
  __shared__ float s_inv[16];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * 16;
  if (threadIdx.x < 16) {
    const int64_t p = p0 + threadIdx.x;
    int64_t srow = 0;
    if (p < n_rows)
      srow = order ? static_cast<int64_t>(static_cast<uint32_t>(order[p]) % static_cast<uint32_t>(n_tokens)) : p;
    s_row[threadIdx.x] = srow;
    if (zero_out && blockIdx.y == 0 && p < n_rows) zero_out[p] = 0u;
  }
  __syncthreads();
  const int n_chunks = n_cols / 8;  // 16-byte chunks of a row
  for (int q = 0; q < 4; ++q) {
    const int r = wave * 4 + q;
    const int64_t p = p0 + r;
    if (p >= n_rows) break;  // wave-uniform
    float amax;
    if (row_amax) {
      amax = __uint_as_float(row_amax[s_row[r]]);
    } else {
      const bf16_t* row = src + s_row[r] * n_cols;
      amax = 0.f;
      for (int c = lane; c < n_chunks; c += kWave)
        amax = fmaxf(amax, absmax_bf16x8(*reinterpret_cast<const u32x4_t*>(row + c * 8)));
      amax = wave_max(amax);
    }
    float inv;
    const float scale = pow2_scale(amax, &inv);
    if (lane == 0) {
      s_inv[r] = inv;
      if (blockIdx.y == 0) dst_scale[p] = scale;
    }
  }
  __syncthreads();
  const int r = lane >> 2, g = lane & 3;
  const int64_t p = p0 + r;
  if (p >= n_rows) return;
  const bf16_t* row = src + s_row[r] * n_cols;
  const float inv = s_inv[r];
  const int n_pieces = n_cols / 64;
  u32x4_t lo[8], hi[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int j = static_cast<int>(blockIdx.y) * 32 + wave + 4 * t;
    if (j < n_pieces) {
      lo[t] = *reinterpret_cast<const u32x4_t*>(row + 64 * j + 8 * g);
      hi[t] = *reinterpret_cast<const u32x4_t*>(row + 64 * j + 32 + 8 * g);
    }
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int j = static_cast<int>(blockIdx.y) * 32 + wave + 4 * t;
    if (j < n_pieces) {
      const int64_t at = (static_cast<int64_t>(j) * n_rows + p) * 64 + g * 16;
      if (dst_lo) {
        u32x2_t ah, al, bh, bl;
        e4m3_codes8_x2(lo[t], inv, ah, al);
        e4m3_codes8_x2(hi[t], inv, bh, bl);
        *reinterpret_cast<u32x4_t*>(dst_q + at) = u32x4_t{ah[0], ah[1], bh[0], bh[1]};
        *reinterpret_cast<u32x4_t*>(dst_lo + at) = u32x4_t{al[0], al[1], bl[0], bl[1]};
      } else {
        const u32x2_t a = e4m3_codes8(lo[t], inv), b = e4m3_codes8(hi[t], inv);
        *reinterpret_cast<u32x4_t*>(dst_q + at) = u32x4_t{a[0], a[1], b[0], b[1]};
      }
    }
  }
}

// combine_kernel with the slot count KS and the split count NS fixed and
// V-wide rows (fp32 partials: 4, bf16 partials: 8, one 16-byte load each):
// all KS * NS loads of an element group are in flight before the first add.
// The adds run in the same order (splits, then slots, then the residual), so
// the result is bit-identical.
template <typename TY, typename TO, int KS, int NS>
__global__ __launch_bounds__(kThreads) void combine_fixed_kernel(const TY* __restrict__ y, const TO* residual,
                                                                 TO* out, int n_tokens, int n_embd,
                                                                 int64_t split_stride) {
  constexpr int V = 16 / sizeof(TY);
  const int64_t total = static_cast<int64_t>(n_tokens) * n_embd;
  for (int64_t i = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * V; i < total;
       i += static_cast<int64_t>(gridDim.x) * kThreads * V) {
    float v[KS][NS][V];
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int q = 0; q < NS; ++q) ldv<V>(y, i + s * total + q * split_stride, v[s][q]);
    float acc[V], p[V];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        float w = v[s][0][j];
#pragma unroll
        for (int q = 1; q < NS; ++q) w += v[s][q][j];
        acc[j] = s == 0 ? w : acc[j] + w;
      }
    }
    if (residual) {
      ldv<V>(residual, i, p);
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] = p[j] + acc[j];
    }
    stv<V>(out, i, acc);
  }
}

// One block per row (grid-stride over rows).  Sum of squares in fp32 (per
// thread, then across the block), rms = sqrt(sum / H + eps), then
// out = (x / rms) * weight, the reference's operation order.  out may alias
// x: a thread writes only the elements it read in both passes.
template <typename T, int V>
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const T* x,
                                                            const T* __restrict__ weight, float eps,
                                                            T* out, int64_t n_rows,
                                                            int n_embd) {
  __shared__ float partial[kThreads / kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  for (int64_t r = blockIdx.x; r < n_rows; r += gridDim.x) {
    const T* xr = x + r * n_embd;
    float ss = 0.f;
    for (int c = threadIdx.x * V; c < n_embd; c += kThreads * V) {
      float v[V];
      ldv<V>(xr, c, v);
#pragma unroll
      for (int j = 0; j < V; ++j) ss += v[j] * v[j];
    }
    ss = wave_sum(ss);
    if (lane == 0) partial[wave] = ss;
    __syncthreads();
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) sum += partial[w];
    __syncthreads();  // partial[] is rewritten by the next row
    const float rms = sqrtf(sum / static_cast<float>(n_embd) + eps);
    for (int c = threadIdx.x * V; c < n_embd; c += kThreads * V) {
      float v[V], w[V];
      ldv<V>(xr, c, v);
      ldv<V>(weight, c, w);
#pragma unroll
      for (int j = 0; j < V; ++j) v[j] = (v[j] / rms) * w[j];
      stv<V>(out + r * n_embd, c, v);
    }
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

namespace {
template <typename TY, typename TO>
void combine_t(const void* y, const void* residual, void* out, int n_tokens, int k, int n_embd, int nsplit,
               int64_t split_stride, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(n_tokens) * n_embd;
  // 4-wide when rows, partial strides and every pointer allow 16/8-byte access.
  const bool vec = n_embd % 4 == 0 && split_stride % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(y) % (4 * sizeof(TY)) == 0 &&
                   reinterpret_cast<uintptr_t>(out) % (4 * sizeof(TO)) == 0 &&
                   reinterpret_cast<uintptr_t>(residual) % (4 * sizeof(TO)) == 0;
  // 16-byte partial loads: 4 fp32 or 8 bf16 per thread
  constexpr int VF = 16 / sizeof(TY);
  const bool vec16 = n_embd % VF == 0 && split_stride % VF == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % (VF * sizeof(TO)) == 0 &&
                     reinterpret_cast<uintptr_t>(residual) % (VF * sizeof(TO)) == 0;
  if (vec16 && k >= 1 && k <= 8 && nsplit >= 1 && nsplit <= 2) {
    using Fn = void (*)(const TY*, const TO*, TO*, int, int, int64_t);
    static constexpr Fn table[8][2] = {
        {combine_fixed_kernel<TY, TO, 1, 1>, combine_fixed_kernel<TY, TO, 1, 2>},
        {combine_fixed_kernel<TY, TO, 2, 1>, combine_fixed_kernel<TY, TO, 2, 2>},
        {combine_fixed_kernel<TY, TO, 3, 1>, combine_fixed_kernel<TY, TO, 3, 2>},
        {combine_fixed_kernel<TY, TO, 4, 1>, combine_fixed_kernel<TY, TO, 4, 2>},
        {combine_fixed_kernel<TY, TO, 5, 1>, combine_fixed_kernel<TY, TO, 5, 2>},
        {combine_fixed_kernel<TY, TO, 6, 1>, combine_fixed_kernel<TY, TO, 6, 2>},
        {combine_fixed_kernel<TY, TO, 7, 1>, combine_fixed_kernel<TY, TO, 7, 2>},
        {combine_fixed_kernel<TY, TO, 8, 1>, combine_fixed_kernel<TY, TO, 8, 2>}};
    hipLaunchKernelGGL(table[k - 1][nsplit - 1], dim3(grid_for(total / VF)), dim3(kThreads), 0, stream,
                       static_cast<const TY*>(y), static_cast<const TO*>(residual), static_cast<TO*>(out), n_tokens,
                       n_embd, split_stride);
    return;
  }
  if (vec)
    hipLaunchKernelGGL((combine_kernel<TY, TO, 4>), dim3(grid_for(total / 4)), dim3(kThreads), 0, stream,
                       static_cast<const TY*>(y), static_cast<const TO*>(residual), static_cast<TO*>(out),
                       n_tokens, k, n_embd, nsplit, split_stride);
  else
    hipLaunchKernelGGL((combine_kernel<TY, TO, 1>), dim3(grid_for(total)), dim3(kThreads), 0, stream,
                       static_cast<const TY*>(y), static_cast<const TO*>(residual), static_cast<TO*>(out),
                       n_tokens, k, n_embd, nsplit, split_stride);
}

template <typename T>
void rms_norm_t(const void* x, const void* w, float eps, void* out, int64_t n_rows, int n_embd,
                hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>(n_rows < 65536 ? n_rows : 65536);
  const bool vec = n_embd % 4 == 0 && reinterpret_cast<uintptr_t>(x) % (4 * sizeof(T)) == 0 &&
                   reinterpret_cast<uintptr_t>(w) % (4 * sizeof(T)) == 0 &&
                   reinterpret_cast<uintptr_t>(out) % (4 * sizeof(T)) == 0;
  if (vec)
    hipLaunchKernelGGL((rms_norm_kernel<T, 4>), dim3(grid), dim3(kThreads), 0, stream, static_cast<const T*>(x),
                       static_cast<const T*>(w), eps, static_cast<T*>(out), n_rows, n_embd);
  else
    hipLaunchKernelGGL((rms_norm_kernel<T, 1>), dim3(grid), dim3(kThreads), 0, stream, static_cast<const T*>(x),
                       static_cast<const T*>(w), eps, static_cast<T*>(out), n_rows, n_embd);
}
}  // namespace

hipError_t launch_combine(const void* y, int y_dtype, const void* residual, void* out, int out_dtype,
                          int n_tokens, int k, int n_embd, int nsplit, int64_t split_stride, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(n_tokens) * n_embd;
  if (total == 0) return hipSuccess;
  if (y_dtype == DT_F32 && out_dtype == DT_F32)
    combine_t<float, float>(y, residual, out, n_tokens, k, n_embd, nsplit, split_stride, stream);
  else if (y_dtype == DT_F32)
    combine_t<float, bf16_t>(y, residual, out, n_tokens, k, n_embd, nsplit, split_stride, stream);
  else if (out_dtype == DT_F32)
    combine_t<bf16_t, float>(y, residual, out, n_tokens, k, n_embd, nsplit, split_stride, stream);
  else
    combine_t<bf16_t, bf16_t>(y, residual, out, n_tokens, k, n_embd, nsplit, split_stride, stream);
  return hipGetLastError();
}

hipError_t launch_rms_norm(const void* x, const void* weight, float eps, void* out, int64_t n_rows, int n_embd,
                           int dtype, hipStream_t stream) {
  if (n_rows == 0 || n_embd == 0) return hipSuccess;
  if (dtype == DT_F32)
    rms_norm_t<float>(x, weight, eps, out, n_rows, n_embd, stream);
  else
    rms_norm_t<bf16_t>(x, weight, eps, out, n_rows, n_embd, stream);
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

hipError_t launch_row_absmax(const void* src, int n_rows, int n_cols, unsigned* amax_out, unsigned* zero_out,
                             int n_zero, hipStream_t stream) {
  if (n_rows <= 0 && (!zero_out || n_zero <= 0)) return hipSuccess;
  if (n_cols <= 0 || n_cols % 8 || reinterpret_cast<uintptr_t>(src) % 16) return hipErrorInvalidValue;
  constexpr int waves = kThreads / kWave;
  const int64_t need = std::max<int64_t>((static_cast<int64_t>(n_rows) + waves - 1) / waves,
                                         (static_cast<int64_t>(n_zero) + kThreads - 1) / kThreads);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(std::max<int64_t>(need, 1), 1 << 16));
  hipLaunchKernelGGL(row_absmax_kernel, dim3(blocks), dim3(kThreads), 0, stream, static_cast<const bf16_t*>(src),
                     n_rows, n_cols, amax_out, zero_out, n_zero);
  return hipGetLastError();
}

hipError_t launch_quantize_rows_kb(const void* src, const int* order, int n_rows, int n_tokens, int n_cols,
                                   const unsigned* row_amax, void* dst_q, float* dst_scale, unsigned* zero_out,
                                   hipStream_t stream, void* dst_lo) {
  if (n_rows <= 0) return hipSuccess;
  if (n_cols <= 0 || n_cols % 64 || n_cols > 16384 || reinterpret_cast<uintptr_t>(src) % 16 ||
      reinterpret_cast<uintptr_t>(dst_q) % 16 || reinterpret_cast<uintptr_t>(dst_lo) % 16 || (order && n_tokens <= 0))
    return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>((static_cast<int64_t>(n_rows) + 15) / 16),
                  static_cast<unsigned>((n_cols / 64 + 31) / 32));
  hipLaunchKernelGGL(quantize_rows_kb_kernel, grid, dim3(kThreads), 0, stream,
                     static_cast<const bf16_t*>(src), order, n_rows, n_tokens, n_cols, row_amax,
                     static_cast<uint8_t*>(dst_q), dst_scale, zero_out, static_cast<uint8_t*>(dst_lo));
  return hipGetLastError();
}

hipError_t launch_gather_rows_kb(const void* src, const int* order, int n_rows, int n_tokens, int n_cols, void* dst,
                                 hipStream_t stream) {
  if (n_rows <= 0 || n_cols <= 0) return hipSuccess;
  if (n_cols % 32 || reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(dst) % 16)
    return hipErrorInvalidValue;
  const int64_t total = (static_cast<int64_t>(n_rows) + 15) / 16 * (n_cols / 32) * kWave;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + kThreads - 1) / kThreads, 1 << 16));
  hipLaunchKernelGGL(gather_rows_kb_kernel, dim3(blocks), dim3(kThreads), 0, stream,
                     static_cast<const bf16_t*>(src), order, n_rows, n_tokens, n_cols, static_cast<bf16_t*>(dst));
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
