// Device-side helpers shared by the gfx950 kernels of the MoE FFN path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fmoe {

typedef uint16_t bf16_t;  // bfloat16 bit pattern in memory
typedef uint8_t f8_t;     // OCP e4m3fn code in memory

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
// Native 16-byte vector for all data movement (HIP's uint4 is a struct whose
// copies lower to memcpy, which keeps arrays of it out of registers).
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

constexpr int kWave = 64;

// ---------------------------------------------------------------- numbers
__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even (gfx950 v_cvt_pk_bf16_f32), NaN stays NaN.
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(bf16_t, b);
}

// s_waitcnt immediate for vmcnt(vm) (0..63), with or without lgkmcnt(0)
// (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8; a
// field at its maximum does not wait).
__host__ __device__ constexpr int wait_vm(int vm, bool lgkm0) {
  return (vm & 15) | ((vm >> 4) << 14) | 0x70 | (lgkm0 ? 0 : 0xF00);
}

// Block barrier that orders LDS accesses only: unlike __syncthreads it does
// not wait for the wave's outstanding global stores.  For blocks whose
// threads exchange data through LDS alone (global memory written before the
// barrier is not read by another thread of the block after it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// gate * silu(up) = g * u / (1 + exp(-u)) (components/activation/swiglu.mlir:37-47)
// for the MFMA kernels, whose SwiGLU output is stored as bf16: the hardware
// reciprocal (1 ulp) stands in for an IEEE division, far below bf16's
// rounding.  The fp32 reference kernel divides exactly.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * (u * __builtin_amdgcn_rcpf(1.f + __expf(-u)));
}

// RoPE of the adjacent pair (x0, x1) = dimensions (2i, 2i+1) of a head of
// size D at position pos: angle pos * freq_scale / freq_base^(2i/D) in
// double precision (components/position/rope.mlir:38-104,
// oracles/position.py:6-50).
// rope_cos_sin gives the pair's (cos, sin) rounded to float, rope_apply the
// rotation; split so a kernel can compute the angles ahead of its data.  The
// rotation's fused multiply-adds are written out so that every kernel that
// applies it rounds the same way (left to the compiler, the contraction of
// a * c - b * s may pick either product).
__device__ __forceinline__ float2 rope_cos_sin(int64_t pos, int i, int D, double freq_base, double freq_scale) {
  const double freq = freq_scale / pow(freq_base, static_cast<double>(2 * i) / D);
  double sn, cs;
  sincos(static_cast<double>(pos) * freq, &sn, &cs);
  return float2{static_cast<float>(cs), static_cast<float>(sn)};
}

__device__ __forceinline__ void rope_apply(float x0, float x1, float2 cs, float& y0, float& y1) {
  y0 = __builtin_fmaf(x0, cs.x, -(x1 * cs.y));
  y1 = __builtin_fmaf(x0, cs.y, x1 * cs.x);
}

__device__ __forceinline__ void rope_pair(float x0, float x1, int64_t pos, int i, int D, double freq_base,
                                          double freq_scale, float& y0, float& y1) {
  rope_apply(x0, x1, rope_cos_sin(pos, i, D, freq_base, freq_scale), y0, y1);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
  bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// Two e4m3fn codes (bytes 0-1 of w, or 2-3 when HI) -> two bf16 packed in a
// dword, low element first.  Exact: every e4m3fn value is a bf16 value.
template <bool HI>
__device__ __forceinline__ uint32_t cvt2_e4m3fn_bf16(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}

// 8 e4m3fn codes in two dwords -> a bf16x8 fragment (same element order).
__device__ __forceinline__ u32x4_t f8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  return u32x4_t{cvt2_e4m3fn_bf16<false>(lo), cvt2_e4m3fn_bf16<true>(lo), cvt2_e4m3fn_bf16<false>(hi),
                 cvt2_e4m3fn_bf16<true>(hi)};
}

// OCP FP8 E4M3 (e4m3fn) code -> float: (8+m) * 2^(e-10) for e>0, m * 2^-9 for
// e=0, NaN for S.1111.111.
__device__ __forceinline__ float e4m3fn_to_f32(uint32_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xFu;
  uint32_t m = c & 7u;
  float mag;
  if (e == 0) {
    mag = static_cast<float>(m) * 0x1p-9f;
  } else if (e == 15 && m == 7) {
    mag = __uint_as_float(0x7FC00000u);
  } else {
    mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return __uint_as_float(__float_as_uint(mag) | s);
}

// float -> e4m3fn code, round to nearest even, finite overflow saturates to
// +-448, NaN -> 0x7F.  Branch-free: both the normal rounding (RNE
// on the 20 dropped mantissa bits, a carry moving into the exponent) and the
// subnormal one (m * 2^-9, m = rint(|x| * 512), where 8 is the smallest
// normal code) are computed and one is selected.
__device__ __forceinline__ uint32_t f32_to_e4m3fn(float x) {
  const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
  const float a = fabsf(x);
  const uint32_t ab = __float_as_uint(a);
  const uint32_t r = ab + 0x7FFFFu + ((ab >> 20) & 1u);
  const uint32_t normal = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
  const uint32_t sub = static_cast<uint32_t>(__builtin_rintf(a * 512.0f));
  uint32_t code = a < 0x1p-6f ? sub : normal;
  code = a >= 448.0f ? 0x7Eu : code;  // also +inf
  return a != a ? 0x7Fu : (sign | code);
}

// Largest |v| of the 8 bf16 values in a 16-byte chunk (NaN ignored).
__device__ __forceinline__ float absmax_bf16x8(const u32x4_t v) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m = fmaxf(m, fabsf(__uint_as_float(v[i] << 16)));
    m = fmaxf(m, fabsf(__uint_as_float(v[i] & 0xFFFF0000u)));
  }
  return m;
}

// ---------------------------------------------------------------- e4m3 activation codes
// 8 bf16 values times inv -> 8 e4m3fn codes in two dwords (element order),
// two values per v_cvt_pk_fp8_f32 (round to nearest even).  The row scale
// keeps every scaled value within +-448, so the instruction's overflow
// behaviour never applies; the codes equal f32_to_e4m3fn's (checked against
// the oracle on every e4m3 value, every tie and its neighbours).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ u32x2_t e4m3_codes8(const u32x4_t v, float inv) {
  uint32_t w[2];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    int c = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_lo(v[2 * d]) * inv, bf16_hi(v[2 * d]) * inv, 0, false);
    c = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_lo(v[2 * d + 1]) * inv, bf16_hi(v[2 * d + 1]) * inv, c, true);
    w[d] = static_cast<uint32_t>(c);
  }
  return u32x2_t{w[0], w[1]};
}

// The same codes as e4m3_codes8 (hi), and in lo the codes of each value's
// remainder, e4m3(v * inv - hi): the two terms hold every bf16 value whose
// scaled magnitude is at least 2^-2 exactly (hi keeps its top 4 significant
// bits, the remainder fits the next 4 within lo's exponent range).  hi is
// decoded back exactly with v_cvt_pk_f32_fp8.
__device__ __forceinline__ void e4m3_codes8_x2(const u32x4_t v, float inv, u32x2_t& hi, u32x2_t& lo) {
  hi = e4m3_codes8(v, inv);
  uint32_t wl[2];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const int h = static_cast<int>(hi[d]);
    const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8(h, false);
    const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8(h, true);
    int c = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_lo(v[2 * d]) * inv - h01[0], bf16_hi(v[2 * d]) * inv - h01[1], 0,
                                            false);
    c = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_lo(v[2 * d + 1]) * inv - h23[0], bf16_hi(v[2 * d + 1]) * inv - h23[1],
                                        c, true);
    wl[d] = static_cast<uint32_t>(c);
  }
  lo = u32x2_t{wl[0], wl[1]};
}

// Power-of-two scale 2^e of a row whose largest magnitude is amax: the
// smallest e with amax / 2^e <= 448 (448 = 1.75 * 2^8), clamped to
// [-126, 126]; 1 for amax = 0.  *inv = 2^-e.  Exact to apply, and each
// value's rounding depends only on the value and its binade.
__device__ __forceinline__ float pow2_scale(float amax, float* inv) {
  if (!(amax > 0.f)) {
    *inv = 1.f;
    return 1.f;
  }
  const uint32_t ab = __float_as_uint(amax);
  int e = static_cast<int>(ab >> 23) - 127 - 8 + ((ab & 0x7FFFFFu) > 0x600000u ? 1 : 0);
  e = min(max(e, -126), 126);
  *inv = __uint_as_float(static_cast<uint32_t>(127 - e) << 23);
  return __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
}

// ---------------------------------------------------------------- waves
// Maximum over each 16-lane row of a wave (DPP row rotations; every lane of
// the row must take part and gets the result).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xF, 0xF, false)));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    int u = __shfl_up(v, o, kWave);
    if (lane >= o) v += u;
  }
  return v;
}

// ---------------------------------------------------------------- tiles
// A grouped-GEMM row tile: rows [row0, row0+rows) of the expert-sorted
// assignment list, all routed to `expert`.
struct TileInfo {
  int expert;
  int row0;
  int rows;
};

// Maps tile number `tile` to its expert and rows, given the permutation
// offsets [n_expert+1] and the tile height bm.  Experts contribute
// ceil(count/bm) tiles each, in expert order.  Every lane of the calling wave
// must participate; all lanes get the same answer.  Returns false when `tile`
// is past the last tile.
__device__ __forceinline__ bool find_tile(const int* __restrict__ offsets, int n_expert,
                                          int bm, int tile, TileInfo* out) {
  const int lane = threadIdx.x & (kWave - 1);
  int base = 0;
  for (int c = 0; c < n_expert; c += kWave) {
    const int e = c + lane;
    int cnt = 0;
    if (e < n_expert) cnt = offsets[e + 1] - offsets[e];
    const int nt = (cnt + bm - 1) / bm;
    const int incl = wave_inclusive_scan(nt);
    const int excl = incl - nt;
    const bool hit = (tile >= base + excl) && (tile < base + incl);
    const uint64_t m = __ballot(hit);
    if (m) {
      const int src = __builtin_ctzll(m);
      const int ee = __shfl(e, src, kWave);
      const int ex = __shfl(excl, src, kWave);
      const int cn = __shfl(cnt, src, kWave);
      const int local = tile - base - ex;
      out->expert = ee;
      out->row0 = offsets[ee] + local * bm;
      out->rows = min(bm, cn - local * bm);
      return true;
    }
    base += __shfl(incl, kWave - 1, kWave);
  }
  return false;
}

}  // namespace fmoe
