// Generic grouped GEMM (SIMT fp32 FMA): any shape, any operand type.
//
// Computes, for every row tile of the expert-sorted assignment list,
//   acc[p, n] = sum_k A[row(p), k] * W_e[n, k]
// which is mul_mat_id's per-assignment mat-vec
// (components/moe/mul_mat_id.mlir:55-94, oracles/moe.py:37-45) with the
// assignments of one expert batched into a GEMM.  Used for fp32 (the
// reference's own dtype), for shapes the MFMA kernels do not tile, and as a
// cross-check of those kernels.
//
// 64x64 output tile per 256-thread block, 4x4 per thread, K in steps of 16
// staged through LDS as fp32.
#include "common.h"
#include "launch.h"

namespace fmoe {
namespace {

constexpr int kBM = 64;
constexpr int kBN = 64;
constexpr int kBK = 16;
constexpr int kThreads = 256;

template <typename T>
__device__ __forceinline__ float to_f32(const T* p, int64_t i);
template <>
__device__ __forceinline__ float to_f32<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float to_f32<bf16_t>(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <>
__device__ __forceinline__ float to_f32<f8_t>(const f8_t* p, int64_t i) { return e4m3fn_to_f32(p[i]); }

template <typename TO>
__device__ __forceinline__ void store(TO* p, int64_t i, float v);
template <>
__device__ __forceinline__ void store<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void store<bf16_t>(bf16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

template <typename TA, typename TW, typename TO, int EPI>
__global__ __launch_bounds__(kThreads) void gemm_generic_kernel(GroupedGemmArgs g) {
  constexpr int NB = EPI == EPI_SWIGLU ? 2 : 1;
  __shared__ float As[kBK][kBM + 4];
  __shared__ float Bs[NB][kBK][kBN + 4];

  TileInfo ti;
  if (!find_tile(g.offsets, g.n_expert, kBM, blockIdx.x, &ti)) return;
  const int n0 = blockIdx.y * kBN;
  const int tid = threadIdx.x;
  const int tx = tid & 15;
  const int ty = tid >> 4;
  const int64_t N = g.N, K = g.K;

  // Loader mapping: row/col (tid >> 2), 4 consecutive k at (tid & 3) * 4.
  const int lr = tid >> 2;
  const int lk = (tid & 3) * 4;
  const TA* a_row = nullptr;
  if (lr < ti.rows) {
    const int p = ti.row0 + lr;
    int64_t r = p;
    if (g.a_mode == A_GATHER_TOKEN)
      r = g.order[p] % g.n_tokens;
    else if (g.a_mode == A_GATHER_FLAT)
      r = g.order[p];
    a_row = static_cast<const TA*>(g.a) + r * g.lda;
  }
  const TW* w_base[NB];
  const int bn = n0 + lr;
  w_base[0] = static_cast<const TW*>(g.w0);
  if (NB == 2) w_base[NB - 1] = static_cast<const TW*>(g.w1);
  const bool bn_ok = bn < N;

  float acc[NB][4][4];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[b][i][j] = 0.f;

  for (int64_t k0 = 0; k0 < K; k0 += kBK) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t k = k0 + lk + j;
      As[lk + j][lr] = (a_row && k < K) ? to_f32(a_row, k) : 0.f;
#pragma unroll
      for (int b = 0; b < NB; ++b)
        Bs[b][lk + j][lr] =
            (bn_ok && k < K) ? to_f32(w_base[b], packed_offset(g.w_format, g.w_dtype, ti.expert, bn, k, N, K)) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; ++kk) {
      float av[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float bv = Bs[b][kk][tx * 4 + j];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[b][i][j] = fmaf(av[i], bv, acc[b][i][j]);
        }
      }
    }
    __syncthreads();
  }

  TO* out = static_cast<TO*>(g.out);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = ty * 4 + i;
    if (r >= ti.rows) continue;
    const int p = ti.row0 + r;
    int64_t orow = p;
    float rw = 1.f;
    if (EPI != EPI_SWIGLU) {
      orow = g.order[p];
      if (EPI == EPI_SCATTER_WEIGHTED) rw = g.route_w[orow];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n >= N) continue;
      float v0 = acc[0][i][j];
      if (g.s0) v0 *= g.s0[static_cast<int64_t>(ti.expert) * N + n];
      float v;
      if (EPI == EPI_SWIGLU) {
        float u = acc[NB - 1][i][j];
        if (g.s1) u *= g.s1[static_cast<int64_t>(ti.expert) * N + n];
        // gate * silu(up), silu(u) = u / (1 + exp(-u))  (swiglu.mlir:37-47)
        v = v0 * (u / (1.f + expf(-u)));
      } else {
        v = v0 * rw;
      }
      store(out, orow * g.ldo + n, v);
    }
  }
}

template <typename TA, typename TW, typename TO>
hipError_t dispatch_epi(const GroupedGemmArgs& g, dim3 grid, hipStream_t s) {
  switch (g.epi) {
    case EPI_SWIGLU:
      hipLaunchKernelGGL((gemm_generic_kernel<TA, TW, TO, EPI_SWIGLU>), grid, dim3(kThreads), 0, s, g);
      break;
    case EPI_SCATTER:
      hipLaunchKernelGGL((gemm_generic_kernel<TA, TW, TO, EPI_SCATTER>), grid, dim3(kThreads), 0, s, g);
      break;
    default:
      hipLaunchKernelGGL((gemm_generic_kernel<TA, TW, TO, EPI_SCATTER_WEIGHTED>), grid, dim3(kThreads), 0, s, g);
      break;
  }
  return hipGetLastError();
}

template <typename TA, typename TW>
hipError_t dispatch_out(const GroupedGemmArgs& g, dim3 grid, hipStream_t s) {
  if (g.out_dtype == DT_F32) return dispatch_epi<TA, TW, float>(g, grid, s);
  return dispatch_epi<TA, TW, bf16_t>(g, grid, s);
}

template <typename TA>
hipError_t dispatch_w(const GroupedGemmArgs& g, dim3 grid, hipStream_t s) {
  if (g.w_dtype == DT_F32) return dispatch_out<TA, float>(g, grid, s);
  if (g.w_dtype == DT_BF16) return dispatch_out<TA, bf16_t>(g, grid, s);
  return dispatch_out<TA, f8_t>(g, grid, s);
}

}  // namespace

hipError_t launch_gemm_generic(const GroupedGemmArgs& g, hipStream_t stream) {
  if (g.n_assign == 0 || g.N == 0) return hipSuccess;
  if (!g.order || !g.offsets || g.epi > EPI_SCATTER_WEIGHTED) return hipErrorInvalidValue;
  if (g.a_kb_rows || g.out_kb_rows) return hipErrorNotSupported;
  // x: row tiles (unbounded count), y: output column tiles.
  const dim3 grid(static_cast<unsigned>(max_row_tiles(g.n_assign, g.n_expert, kBM)),
                  static_cast<unsigned>((g.N + kBN - 1) / kBN));
  if (g.act_dtype == DT_F32) return dispatch_w<float>(g, grid, stream);
  return dispatch_w<bf16_t>(g, grid, stream);
}

}  // namespace fmoe
