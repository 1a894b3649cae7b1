// Shared types/helpers of the NS5 kernels and the launcher of the persistent
// 256-block kernels (ns5_stream.hip), used by the dispatcher in ns5.hip.
#pragma once

#include <algorithm>
#include <utility>

#include "common.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// x -> bf16(x * s) for 8 packed bf16 values.
HM_DEV u32x4_t scale8(u32x4_t v, float s) {
  u32x4_t o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float lo = bf16_to_f32(v[k] & 0xffffu) * s;
    const float hi = __uint_as_float(v[k] & 0xffff0000u) * s;
    o[k] = pack2(f32_to_bf16(lo), f32_to_bf16(hi));
  }
  return o;
}

HM_DEV uint32_t half16(uint32_t w, int h) { return h ? (w >> 16) : (w & 0xffffu); }

// Persistent streamed-operand 256-block path (ns5_stream.hip): mp, np
// multiples of 256. Scales x in place (X0), then runs `steps` iterations on
// `cnt` tiles, ping-ponging X between x and y.
bool ns5_stream_supported(int mp, int np);
void ns5_stream_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                    float a, float b, float c, uint16_t* wsA, uint16_t* wsB, hipStream_t s);
