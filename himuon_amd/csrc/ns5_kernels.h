// Shared types/helpers of the NS5 kernels and the launchers of the 256-block
// variants (ns5_big.hip), used by the dispatcher in ns5.hip.
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

// Persistent NT-GEMM path (ns5_nt.hip): mp, np multiples of 256. Runs `steps`
// iterations on `cnt` tiles, ping-ponging X between (x, xt) and (y, yt).
bool ns5_nt_supported(int mp, int np);
void ns5_nt_run(uint16_t* x, uint16_t* xt, uint16_t* y, uint16_t* yt, const float* inv,
                int64_t cnt, int mp, int np, int steps, float a, float b, float c, uint16_t* wsA,
                uint16_t* wsB, hipStream_t s);

// Persistent 256-block path with direct-to-LDS operand loads (ns5_persist.hip):
// mp, np multiples of 256. Scales x in place (X0), then runs `steps`
// iterations on `cnt` tiles, ping-ponging X between x and y.
bool ns5_pk_supported(int mp, int np);
void ns5_pk_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                float a, float b, float c, uint16_t* wsA, uint16_t* wsB, hipStream_t s);

// Persistent streamed-operand 256-block path (ns5_stream.hip): mp, np
// multiples of 256. Scales x in place (X0), then runs `steps` iterations on
// `cnt` tiles, ping-ponging X between x and y.
bool ns5_stream_supported(int mp, int np);
void ns5_stream_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                    float a, float b, float c, uint16_t* wsA, uint16_t* wsB, hipStream_t s);

// Persistent two-workgroups-per-CU path (ns5_duo.hip): mp a multiple of 256,
// np of 128. Scales x in place (X0), then runs `steps` iterations on `cnt`
// tiles, ping-ponging X between x and y.
bool ns5_duo_supported(int mp, int np);
void ns5_duo_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                 float a, float b, float c, uint16_t* wsA, uint16_t* wsB, hipStream_t s);

// Dataflow variant of the same kernels (ns5_duo.hip): one persistent launch
// for all iterations; windows of `window` tiles are processed XCD-locally.
// `counters` is the workspace tail of ns5_flow_counter_bytes(cnt) bytes.
size_t ns5_flow_counter_bytes(int64_t cnt);
void ns5_flow_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                  float a, float b, float c, uint16_t* wsA, uint16_t* wsB, int* counters, int window,
                  hipStream_t s);

// Persistent 512x512-tile path (ns5_t512.hip): mp == np == 512. Scales x in
// place (X0), then runs `steps` iterations on `cnt` tiles, ping-ponging X
// between x and y.
bool ns5_t512_supported(int mp, int np);
void ns5_t512_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int steps, float a, float b, float c,
                  uint16_t* wsA, uint16_t* wsB, hipStream_t s);

// 256x256-block stages (M, N, K multiples of 256 / 64).
void ns5_launch_gram256(const uint16_t* S, int64_t s_bs, int ldS, uint16_t* C, int64_t c_bs,
                        int ldC, const float* inv, int M, int K, int64_t ntiles, float alpha,
                        float beta, hipStream_t s);
void ns5_launch_apply256(const uint16_t* Bm, int64_t b_bs, const uint16_t* X, int64_t x_bs,
                         uint16_t* Y, int64_t y_bs, const float* inv, int M, int N, int64_t ntiles,
                         float a, hipStream_t s);
