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

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) const u32x4_t lds_cu32x4;
typedef __attribute__((address_space(3))) const u32x2_t lds_cu32x2;
typedef __attribute__((address_space(3))) u32x2_t lds_u32x2;

// v_mfma_f32_32x32x16_bf16: 8 bf16 of A (row l%32) and of B (column l%32) per lane,
// k = 8 (l/32) .. + 7; the 32x32 fp32 result has row 8 (r/4) + 4 (l/32) + r%4,
// column l%32 in register r of lane l.
HM_DEV f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// bf16 pair (RNE, hardware v_cvt_pk_bf16_f32): lo in bits 0..15.
HM_DEV uint32_t pk_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t r;
  r[0] = (__bf16)lo;
  r[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

// x -> bf16(x * s) for 8 packed bf16 values with the hardware RNE
// conversion (equal to scale8 for every finite product).
HM_DEV u32x4_t scale8_rne(u32x4_t v, float s) {
  u32x4_t o;
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = pk_bf16(__uint_as_float(v[k] << 16) * s, __uint_as_float(v[k] & 0xffff0000u) * s);
  return o;
}

// p[i] for a wave-uniform p and i, read with a scalar load (written by an
// earlier launch). The compiler makes a vector load of it in kernels that
// also store to global memory, and the first use of that load then waits for
// vmcnt(0): for every direct-to-LDS operand load in flight, which the
// compiler does not count. The scalar load is waited for with lgkmcnt.
HM_DEV float uniform_load_f32(const float* p, int64_t i) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)i);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)i >> 32));
  const float* a = p + (int64_t)(((uint64_t)hi << 32) | lo);
  float v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(a) : "memory");
  return v;
}

// s_waitcnt with vmcnt = N (expcnt and lgkmcnt at their maxima) / lgkmcnt = N.
template <int N>
HM_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
template <int N>
HM_DEV void wait_lgkm() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __builtin_amdgcn_s_waitcnt(0xC07F | (N << 8));
}

// ds_read_b64_tr_b16 at an LDS byte address. Issued as inline assembly: the
// compiler cannot tell these reads apart from the direct-to-LDS loads in
// flight and would put a vmcnt(0) wait (draining the operand stream) before
// the builtin. The result is only valid after an explicit lgkmcnt wait.
// OFF: the instruction's immediate byte offset (0 .. 65535).
template <int OFF = 0>
HM_DEV u32x2_t ds_read_tr16(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "DS offset range");
  u32x2_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return r;
}

// Workgroup barrier for LDS reuse: this wave's LDS operations are complete;
// global memory operations (including direct-to-LDS loads) may still be in
// flight and are waited for explicitly with vmcnt. (__syncthreads() lowers
// to a fence that waits for every outstanding load and store, which would
// drain the operand stream at each barrier.)
HM_DEV void lds_barrier() {
  wait_lgkm<0>();
  asm volatile("s_barrier" ::: "memory");
}

// Direct-to-LDS 16-byte load: lane l's 16 bytes from gptr land at LDS byte
// lds_wave + 16 l (lds_wave is wave-uniform, passed in M0). Issued as inline
// assembly: the compiler models the builtin as a flat access to both global
// memory and LDS and, while one is pending, forces lgkmcnt(0)/vmcnt(0) waits
// before unrelated LDS reads. Completion is tracked by vmcnt (in issue order
// with the other vector loads) and waited for explicitly.
HM_DEV void dma16(const void* gptr, uint32_t lds_wave) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(gptr), "s"(__builtin_amdgcn_readfirstlane(lds_wave))
      : "memory", "m0");
}

// DPP quad permutations.
HM_DEV uint32_t quad_swap2(uint32_t v) {  // lane ^ 2
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
}
HM_DEV uint32_t quad_swap1(uint32_t v) {  // lane ^ 1
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
}

// 4x4 bf16 transpose across a lane quad: lane k holds row k as (w0, w1) =
// columns (0,1), (2,3); returns column k as rows (0,1), (2,3).
HM_DEV u32x2_t quad_transpose(u32x2_t w, int k) {
  const uint32_t send_a = (k < 2) ? w[1] : w[0];
  const uint32_t recv_a = quad_swap2(send_a);
  const uint32_t x = (k < 2) ? w[0] : recv_a;
  const uint32_t y = (k < 2) ? recv_a : w[1];
  const bool odd = k & 1;
  const uint32_t send_b = odd ? ((x & 0xffffu) | (y << 16)) : ((x >> 16) | (y & 0xffff0000u));
  const uint32_t r = quad_swap1(send_b);
  u32x2_t o;
  if (odd) {
    o[0] = (r & 0xffffu) | (x & 0xffff0000u);
    o[1] = (r >> 16) | (y & 0xffff0000u);
  } else {
    o[0] = (x & 0xffffu) | (r << 16);
    o[1] = (y & 0xffffu) | (r & 0xffff0000u);
  }
  return o;
}


// The untile with WD/LR fused into the last NS iteration of 512 x 512 tiles
// (himuon_ns5_untile_apply): instead of storing X', the fused kernel's
// epilogue applies each value u = upd_scale X' of tile tile0 + t (t the tile's
// index in the launch) to its parameter element in place, as
// himuon_untile_apply does (tiles not transposed: tile_h <= tile_w).
struct BaUntile {
  const HimuonParamDesc* params;  // device descriptor table of the bucket
  int n_params;
  int64_t tile0;                  // bucket tile index of the launch's tile 0
  int tile_h, tile_w;
  int param_dtype;
  const float* sa;                // device (scale, alpha) per param group, 2 x HIMUON_APPLY_MAX_GROUPS floats
  int32_t* rec;                   // device scratch of 16 int32 per tile of the launch (set by ns5_stream_run)
};

// Persistent streamed-operand 256-block path (ns5_stream.hip): mp, np
// multiples of 256. Runs `steps` iterations on `cnt` tiles from the raw x
// (the first iteration scales X0 = bf16(x inv) on load), ping-ponging X
// between x and y. round_once: the third product
// rounds bf16(B X + a X) once (the 2-D form) instead of bf16(bf16(B X) + a X).
// fused_ba: the second and third products run as one kernel (ns5_ba.hip;
// mp == np == 512), wsB unused. Returns 0, or HIMUON_EINVAL (nothing
// launched) when cnt is too large for the fused kernel.
bool ns5_stream_supported(int mp, int np);
// untile (fused_ba only; steps >= 2): the last iteration applies the untile
// with WD/LR instead of storing its result.
int ns5_stream_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                    float a, float b, float c, bool round_once, bool fused_ba, uint16_t* wsA, uint16_t* wsB,
                    hipStream_t s, const BaUntile* untile = nullptr);

// Fused B = bf16(c A A^T + b A), Y = bf16(bf16(B X) + a X) (ns5_ba.hip) on
// `cnt` 512 x 512 tiles: A from the first product, X -> Y (Y != X). xinv
// non-null: X is the raw tile and X0 = bf16(X xinv[tile]) is used in its
// place (the first iteration). Its work items are (tile, 128-row panel)
// with 32-bit indices: cnt must lie in 1 .. kBaMaxTiles, else nothing is
// launched and false returned.
constexpr int64_t kBaMaxTiles = (int64_t(1) << 29) - 1;
bool ns5_ba_supported(int mp, int np);
// untile non-null: Y is not written; the results update the parameters
// (xinv must be null, param_dtype fp32 or bf16; false otherwise).
bool ns5_ba_run(const uint16_t* A, const uint16_t* X, uint16_t* Y, const float* xinv, int64_t cnt, float a,
                float b, float c, bool round_once, hipStream_t s, const BaUntile* untile = nullptr);

// One NS product over `ntiles` batch entries on the 256-block stream kernels
// (M, N, K multiples of 256; row pitches in elements, batch strides):
//   mode 0: C = bf16(P P^T)                      P: M x K, C: M x M
//   mode 1: C = bf16(alpha P P^T + beta R)       R = P, K = M
//   mode 2: C = bf16(bf16(P Q) + beta R)         P: M x K (K = M), Q, R, C: M x N
//           (bf16(P Q + beta R) with round_once)
void ns_stream_product(int mode, const uint16_t* P, int64_t p_bs, int ldp, const uint16_t* Q, int64_t q_bs,
                       int ldq, const uint16_t* R, int64_t r_bs, int ldr, uint16_t* C, int64_t c_bs, int ldc,
                       int M, int N, int K, int64_t ntiles, float alpha, float beta, bool round_once,
                       hipStream_t s);

// Fused LDS-resident path (ns5_lds.hip): mp == 128, np = 128 or 256. Runs
// `steps` >= 1 iterations of `cnt` tiles in one launch; reads X from x and
// leaves the result in x (even `steps`) or y (odd), as the other paths do.
// The whole step of a bucket of NS tiles with tile_h <= tile_w <= 128 in one
// launch (ns5_lds.hip): momentum + gather + normaliser + NS5 + untile with
// WD/LR, on bucket tiles tile_begin .. tile_begin + cnt - 1; grad/momentum
// dtype `dtype`, parameter dtype `param_dtype` (fp32 or bf16 each).
bool lds_step_supported(int tile_h, int tile_w, int dtype, int param_dtype);
void lds_step_run(const HimuonParamDesc* params, int n_params, int64_t tile_begin, int64_t cnt, int tile_h,
                  int tile_w, int dtype, int param_dtype, int steps, float a, float b, float c, float eps,
                  bool round_once, const float* sa, hipStream_t s);
// NS tiles with m <= 64 real rows in a 128-row padded buffer (ns5_small.hip):
// the tile's rows 0 .. me - 1 (me = 16, 32 or 64 >= m) iterate in LDS, one
// workgroup per tile; np = 128 (me = 64), up to 1024 (32) or 2048 (16). Reads
// x, leaves the result's me rows in x (even `steps`) or y (odd) and touches no
// other row. False (nothing launched) for an unsupported geometry.
bool ns5_small_supported(int m, int mp, int np);
bool ns5_small_run(const uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int m, int np, int steps,
                   float a, float b, float c, bool round_once, hipStream_t s);
bool ns5_lds_supported(int mp, int np);
void ns5_lds_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                 float a, float b, float c, bool round_once, hipStream_t s);
