// Shared device helpers for the HiMuon gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/himuon_hip.h"

#define HM_DEV __device__ __forceinline__
#define HM_HD __host__ __device__ __forceinline__

// ---------------------------------------------------------------------------
// bf16 / fp16 <-> fp32. Rounding is round-to-nearest-even with quiet NaNs,
// the rounding torch's `.to(torch.bfloat16)` performs.
// ---------------------------------------------------------------------------
HM_DEV float bf16_to_f32(uint32_t v) { return __uint_as_float(v << 16); }

// The hardware conversion (v_cvt_pk_bf16_f32, round to nearest even) and the
// canonical quiet NaN 0x7fc0 for every NaN input.
HM_DEV uint32_t f32_to_bf16(float f) {
  const __bf16 h = (__bf16)f;
  const uint32_t b = (uint32_t)__builtin_bit_cast(uint16_t, h);
  return f != f ? 0x7fc0u : b;
}

// Round an fp32 value to the nearest bf16 and return it as fp32.
HM_DEV float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

HM_DEV float f16_to_f32(uint16_t v) {
  _Float16 h;
  __builtin_memcpy(&h, &v, 2);
  return (float)h;
}

// fp32 -> fp16 bits, round to nearest even, in integer arithmetic (the
// compiler cannot merge it with neighbouring fp32 operations).
HM_DEV uint16_t f32_to_f16(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);   // NaN
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // >= 65520 -> inf
  if (ax >= 0x38800000u) {                                   // normal fp16
    const uint32_t r = ax - 0x38000000u;                     // rebias 127 -> 15
    return (uint16_t)(sign | ((r + 0x0fffu + ((r >> 13) & 1u)) >> 13));
  }
  const uint32_t e = ax >> 23;  // subnormal fp16 (or zero): units of 2^-24
  if (e < 102) return (uint16_t)sign;
  const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
  const uint32_t sh = 126 - e;  // 14..24
  const uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
  return (uint16_t)(sign | (q + ((rem > half) || (rem == half && (q & 1u)))));
}

// p + alpha * u rounded ONCE to fp16 (u and p already fp16 values): torch's
// in-place add of an fp32 tensor into an fp16 one evaluates it as a fused
// mixed-precision multiply-add with a single rounding. The exact value
// (a 35-bit product plus an fp16 term) is formed in double; converting it to
// fp32 with round-to-odd and then to fp16 with round-to-nearest-even rounds it
// once, since fp32 keeps more than two bits beyond fp16's precision.
HM_DEV float fma_f16_once(float alpha, float u, float p) {
  const double t = __builtin_fma((double)alpha, (double)u, (double)p);
  float r = __double2float_rz(t);
  if ((double)r != t) r = __uint_as_float(__float_as_uint(r) | 1u);
  return f16_to_f32(f32_to_f16(r));
}

// Load / store one element of a gradient-typed tensor as fp32.
template <int DT>
HM_DEV float load_elem(const void* p, int64_t i) {
  if constexpr (DT == HIMUON_DTYPE_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (DT == HIMUON_DTYPE_BF16) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
}

template <int DT>
HM_DEV float round_to(float f) {
  if constexpr (DT == HIMUON_DTYPE_F32) {
    return f;
  } else if constexpr (DT == HIMUON_DTYPE_BF16) {
    return round_bf16(f);
  } else {
    return f16_to_f32(f32_to_f16(f));
  }
}

template <int DT>
HM_DEV void store_elem(void* p, int64_t i, float v) {
  if constexpr (DT == HIMUON_DTYPE_F32) {
    static_cast<float*>(p)[i] = v;
  } else if constexpr (DT == HIMUON_DTYPE_BF16) {
    static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16(v);
  } else {
    static_cast<uint16_t*>(p)[i] = f32_to_f16(v);
  }
}

// Pack two bf16 bit patterns (lo, hi) into one dword.
HM_DEV uint32_t pack2(uint32_t lo, uint32_t hi) { return (lo & 0xffffu) | (hi << 16); }

// 8 consecutive elements of a gradient-typed row, as fp32.
template <int DT>
HM_DEV void load8(const void* base, int64_t off, float v[8]) {
  if constexpr (DT == HIMUON_DTYPE_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + off);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == HIMUON_DTYPE_BF16) {
        v[2 * k] = bf16_to_f32(w[k] & 0xffffu);
        v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      } else {
        v[2 * k] = f16_to_f32((uint16_t)(w[k] & 0xffffu));
        v[2 * k + 1] = f16_to_f32((uint16_t)(w[k] >> 16));
      }
    }
  }
}

template <int DT>
HM_DEV void store8(void* base, int64_t off, const float v[8]) {
  if constexpr (DT == HIMUON_DTYPE_F32) {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(base) + off);
    p[0] = make_float4(v[0], v[1], v[2], v[3]);
    p[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == HIMUON_DTYPE_BF16) {
        w[k] = pack2(f32_to_bf16(v[2 * k]), f32_to_bf16(v[2 * k + 1]));
      } else {
        w[k] = pack2(f32_to_f16(v[2 * k]), f32_to_f16(v[2 * k + 1]));
      }
    }
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + off) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <int DT>
HM_DEV bool aligned16(const void* base, int64_t off) {
  constexpr int es = (DT == HIMUON_DTYPE_F32) ? 4 : 2;
  return ((reinterpret_cast<uintptr_t>(base) + (uintptr_t)off * es) & 15u) == 0;
}

// ---------------------------------------------------------------------------
// Work-item -> XCD mapping. MI355X dispatches consecutive workgroups
// round-robin over its 8 XCDs, each with a private L2. Items that share data
// (the blocks of one NS tile) are given consecutive item numbers; this maps
// workgroup b to item (b % 8) * per_xcd + b / 8 so that each XCD walks one
// contiguous range of items and a tile's blocks share an L2.
// Grid size must be 8 * per_xcd, per_xcd = ceil(total / 8).
// ---------------------------------------------------------------------------
constexpr int kNumXcd = 8;

HM_DEV int64_t xcd_item(int64_t total) {
  const int64_t per_xcd = (total + kNumXcd - 1) / kNumXcd;
  return (int64_t)(blockIdx.x % kNumXcd) * per_xcd + blockIdx.x / kNumXcd;
}

inline int64_t xcd_grid(int64_t total) {
  const int64_t per_xcd = (total + kNumXcd - 1) / kNumXcd;
  return per_xcd * kNumXcd;
}

// Find the parameter owning tile t: the last p with params[p].tile0 <= t.
HM_DEV int find_param(const HimuonParamDesc* __restrict__ params, int n_params, int64_t t) {
  int lo = 0, hi = n_params - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (params[mid].tile0 <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Wave/block reduction of a float (deterministic order).
HM_DEV float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int NT>
HM_DEV float block_sum(float v, float* red /* >= NT/64 floats of LDS */) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
  if (threadIdx.x == 0) {
    for (int i = 0; i < NT / 64; ++i) s += red[i];
  }
  return s;  // valid in thread 0 only
}
