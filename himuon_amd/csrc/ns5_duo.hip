// Persistent NS5 stage kernels that run two workgroups per CU, so that one
// workgroup's epilogue (conversion, staging and stores of its output block)
// and its operand-stream start-up overlap the other's MFMA work:
//
//   GramA : C = A = bf16(X X^T)            P = Q = X (rows, K = n)   lower blocks + mirror
//   GramB : C = B = bf16(c A A^T + b A)    P = Q = A (rows, K = m)   lower blocks + mirror
//   Apply : C = X' = bf16(bf16(B X) + a X) P = B (rows, K = m), Q = X read as [k][j]
// (ns5_smem.py:89-101, XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88).
//
// Work item: a 256 (i) x 128 (j) output block. A workgroup is 4 waves in a
// 2 x 2 grid, each wave a 128 x 64 sub-block of 4 x 2 v_mfma_f32_32x32x16_bf16
// tiles (128 fp32 accumulators per lane), so two workgroups fit a CU's
// registers (256 per lane) and LDS (2 x 72 KiB).
//
// Operand stream: K advances in units of 32. Each unit (P: 256 rows x 64 B,
// Q: 128 rows x 64 B, or for Apply 32 k-rows x 256 B of X) goes straight from
// global memory into a 24 KiB slot of a 3-slot LDS ring
// (global_load_lds_dwordx4, 1 KiB per wave instruction), two units ahead of
// the MFMAs. Lane l of a direct load writes LDS bytes 16 l .. 16 l + 15 of the
// wave's KiB, so bank spreading is done by choosing which 16-byte source chunk
// each lane fetches (an XOR swizzle of the chunk index by row).
//
// MFMA operands are swapped (A operand = rows j, B operand = rows i), so lane
// l holds C[i = l%32][j = 8q + 4(l/32) .. + 3] of each 32x32 tile. The
// epilogue reads its elementwise operand R (A for GramB, X for Apply) from
// global memory in that layout, stages the bf16 result in the ring's LDS and
// writes it with row-contiguous 16-byte stores. For the Gram products the
// output is symmetric: an item covers 128-blocks (2p, c) and (2p + 1, c) with
// c <= 2p + 1; each wave writes its 128-block if it is on or below the
// diagonal and, below it, also the mirrored block (a 4x4 transpose across
// each lane quad restages it as rows of C^T).
#include "ns5_kernels.h"

namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) const u32x4_t lds_cu32x4;
typedef __attribute__((address_space(3))) u32x2_t lds_u32x2;

constexpr int NT = 256;
constexpr int BI = 256;                    // item rows (i)
constexpr int BJ = 128;                    // item columns (j)
constexpr int BK = 32;                     // K per stream unit
constexpr int PBYTES = BI * BK * 2;        // 16 KiB: P panel of one unit
constexpr int SLOT = PBYTES + BJ * BK * 2; // + 8 KiB Q panel
constexpr int NSLOT = 3;
constexpr int LDS_BYTES = NSLOT * SLOT;    // 72 KiB
constexpr int LP = 4, LQ = 2, L = LP + LQ; // direct loads per wave per unit
constexpr int WSTAGE = 16384;              // bf16 staging bytes per wave (128 x 64)

enum { kGramA = 0, kGramB = 1, kApply = 2 };

struct DuoArgs {
  const uint16_t* P; int64_t p_bs; int ldp;    // rows i, k-contiguous
  const uint16_t* Q; int64_t q_bs; int ldq;    // Gram: rows j, k-contiguous; Apply: X [k][j]
  const uint16_t* R; int64_t r_bs; int ldr;    // epilogue operand [i][j] (A or X)
  uint16_t* C; int64_t c_bs; int ldc;          // output [i][j]
  int M, N, K;
  int64_t ntiles;
  float alpha, beta;                           // GramB: c, b; Apply: beta = a
};

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

// Workgroup barrier for LDS reuse: this wave's LDS operations are complete;
// global memory operations (including direct-to-LDS loads) may still be in
// flight and are waited for explicitly with vmcnt.
HM_DEV void lds_barrier() {
  wait_lgkm<0>();
  asm volatile("s_barrier" ::: "memory");
}

// Direct-to-LDS 16-byte load: lane l's 16 bytes from gptr land at LDS byte
// lds_wave + 16 l (lds_wave is wave-uniform, passed in M0). Inline assembly,
// so that the compiler does not put vmcnt(0) waits before unrelated LDS reads;
// completion is tracked by vmcnt and waited for explicitly.
HM_DEV void dma16(const void* gptr, uint32_t lds_wave) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(gptr), "s"(__builtin_amdgcn_readfirstlane(lds_wave))
      : "memory", "m0");
}

// ds_read_b64_tr_b16 at an LDS byte address (valid after an lgkmcnt wait).
// Within 16 lanes, lane 4a + b receives element b of the 8-byte rows
// addressed by lanes a, a + 4, a + 8 and a + 12.
HM_DEV u32x2_t ds_read_tr16(uint32_t addr) {
  u32x2_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

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

// Chunk swizzles (16-byte chunk index XOR a function of the row):
//  P/Q row panels (64-byte rows): 16 consecutive rows of one chunk spread
//  over distinct bank groups;
//  X panel of Apply (256-byte k-rows): the transposing reads of 4 k-rows x
//  64 bytes land in the 4 distinct 64-byte bank groups;
//  output staging (128-byte rows, 8 chunks) and mirror staging (256-byte
//  rows): the 8-byte writes of one instruction spread over the banks.
HM_DEV int swz_p(int r) { return (((r >> 1) ^ (r >> 3)) & 1) | (((r >> 2) & 1) << 1); }
HM_DEV int swz_q(int r) { return 4 * (r & 3); }
HM_DEV int swz_o(int r) { return (r >> 1) & 7; }
HM_DEV int swz_m(int r) { return 4 * (r & 3); }

// One 256 x 128 output block C[tile][p-block][c-block].
template <int MODE, int NKC>
__device__ __forceinline__ void duo_item(const DuoArgs& g, lds_u8* lds, int64_t tile, int p, int c) {
  constexpr bool kTr = MODE == kApply;
  // The lane index is made opaque per item so that per-lane addresses are
  // recomputed for each item instead of being hoisted out of the persistent
  // loop (where they would not fit in registers).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  const int nk = NKC > 0 ? NKC : g.K / BK;
  const int row0 = p * BI, col0 = c * BJ;

  // ---- loaders -------------------------------------------------------------
  // P unit (256 rows x 64 B): wave instruction i fills rows 16 n .. 16 n + 15,
  // n = 4 i + wave; lane l lands at row 16 n + l/4, position l%4, fetching
  // chunk (l%4) ^ swz_p(row) (row & 15 = l/4). Q unit of the Gram products:
  // the same for 128 rows j (i = 0, 1).
  const int prl = lane >> 2;
  const int pch = (lane & 3) ^ swz_p(prl);
  const uint16_t* psrc = g.P + tile * g.p_bs + (int64_t)(row0 + 16 * wave + prl) * g.ldp + pch * 8;
  const int64_t pstep = 64 * (int64_t)g.ldp;
  const uint16_t* qsrc;
  int64_t qstep, qunit;
  if constexpr (kTr) {
    // X unit (32 k-rows x 256 B): instruction i fills k-rows 4 n .. 4 n + 3,
    // n = 4 i + wave; lane l lands at k-row 4 n + l/16, position l%16,
    // fetching chunk (l%16) ^ swz_q(k-row).
    const int xr = 4 * wave + (lane >> 4);
    const int xc = (lane & 15) ^ swz_q(xr);
    qsrc = g.Q + tile * g.q_bs + (int64_t)xr * g.ldq + col0 + xc * 8;
    qstep = 16 * (int64_t)g.ldq;
    qunit = BK * (int64_t)g.ldq;
  } else {
    qsrc = g.Q + tile * g.q_bs + (int64_t)(col0 + 16 * wave + prl) * g.ldq + pch * 8;
    qstep = 64 * (int64_t)g.ldq;
    qunit = BK;
  }
  const uint32_t wdst = (uint32_t)(uintptr_t)lds + wave * 1024;
  auto issue = [&](int v) {
    const uint32_t d = wdst + (v % NSLOT) * SLOT;
#pragma unroll
    for (int i = 0; i < LP; ++i) dma16(psrc + i * pstep + v * BK, d + i * 4096);
#pragma unroll
    for (int i = 0; i < LQ; ++i) dma16(qsrc + i * qstep + v * qunit, d + PBYTES + i * 4096);
  };

  // ---- MFMA fragments of unit v, sub-step ks -------------------------------
  // B operand (rows i = wm*128 + 32 t + l32 of P): k-chunk 2 ks + hi. A
  // operand (rows j = wn*64 + 32 t + l32): the same from Q for the Gram
  // products; for Apply two transposing reads of the X panel give lane l
  // column j, k = 16 ks + 8 hi + 0..7.
  const int sp = swz_p(l32 & 15);
  const int prow = (wm * 128 + l32) * 64, qrow = (wn * 64 + l32) * 64;
  const int r16 = lane & 15, ta = r16 >> 2, tb = r16 & 3;
  const int tr_row = 8 * hi + ta;
  const int tr_chunk = wn * 8 + 2 * ((lane >> 4) & 1) + (tb >> 1);
  const int tr_sub = (tb & 1) * 8;
  const int tr_s = swz_q(ta);
  auto frags = [&](int v, int ks, u32x4_t(&fa)[2], u32x4_t(&fb)[4]) {
    const lds_u8* s = lds + (v % NSLOT) * SLOT;
    const int pos = ((2 * ks + hi) ^ sp) * 16;
#pragma unroll
    for (int t = 0; t < 4; ++t) fb[t] = *reinterpret_cast<lds_cu32x4*>(s + prow + t * 2048 + pos);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if constexpr (kTr) {
        const uint32_t off = (uint32_t)(uintptr_t)s + PBYTES + (16 * ks + tr_row) * 256 +
                             (((tr_chunk + 4 * t) ^ tr_s) * 16) + tr_sub;
        const u32x2_t l2 = ds_read_tr16(off), u2 = ds_read_tr16(off + 4 * 256);
        fa[t] = u32x4_t{l2[0], l2[1], u2[0], u2[1]};
      } else {
        fa[t] = *reinterpret_cast<lds_cu32x4*>(s + PBYTES + qrow + t * 2048 + pos);
      }
    }
  };

  f32x16_t acc[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;
  auto mma = [&](const u32x4_t(&fa)[2], const u32x4_t(&fb)[4]) {
#pragma unroll
    for (int tj = 0; tj < 2; ++tj)
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
  };

  // ---- K loop ----------------------------------------------------------------
  // Unit u lives in slot u % 3. At the top of unit u + 1 each wave waits for
  // its own loads of that unit; the barrier then publishes it and frees slot
  // u % 3 (every wave holds its unit-u fragments in registers), which receives
  // unit u + 3. The second half of unit u's MFMAs runs after the barrier,
  // covering the first fragment reads of unit u + 1.
  lds_barrier();  // the previous item's staging reads are done
  issue(0);
  if (nk > 1) issue(1);
  if (nk > 1) wait_vm<L>(); else wait_vm<0>();
  lds_barrier();
  if (nk > 2) issue(2);
  u32x4_t fa0[2], fb0[4], fa1[2], fb1[4];
  frags(0, 0, fa0, fb0);
  wait_lgkm<0>();
  __builtin_amdgcn_sched_barrier(0);
  frags(0, 1, fa1, fb1);
  __builtin_amdgcn_sched_barrier(0);
  auto unit = [&](int u) {
    mma(fa0, fb0);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm<0>();  // second-half fragments of unit u
    if (u + 2 < nk) wait_vm<L>(); else wait_vm<0>();  // unit u + 1 has landed
    lds_barrier();
    if (u + 3 < nk) issue(u + 3);
    frags(u + 1, 0, fa0, fb0);
    __builtin_amdgcn_sched_barrier(0);
    mma(fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm<0>();  // first-half fragments of unit u + 1
    frags(u + 1, 1, fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (NKC > 0) {
#pragma unroll
    for (int u = 0; u + 1 < NKC; ++u) unit(u);
  } else {
    for (int u = 0; u + 1 < nk; ++u) unit(u);
  }
  mma(fa0, fb0);
  __builtin_amdgcn_sched_barrier(0);
  wait_lgkm<0>();
  mma(fa1, fb1);

  // ---- epilogue --------------------------------------------------------------
  // This wave's sub-block: rows i = row0 + wm*128 + 32 ti + l32, columns
  // j = col0 + wn*64 + 32 tj + 8 q + 4 hi .. + 3.
  const int ib = row0 + wm * 128, jb = col0 + wn * 64;
  bool write = true, mirror = false;
  if constexpr (MODE != kApply) {
    const int r128 = 2 * p + wm;  // 128-block row of this wave (column block c)
    write = r128 >= c;
    mirror = r128 > c;
  }
  u32x2_t out[4][2][4];
  if constexpr (MODE == kGramA) {
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int tj = 0; tj < 2; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x16_t& v = acc[tj][ti];
          out[ti][tj][q] = u32x2_t{pk_bf16(v[4 * q], v[4 * q + 1]), pk_bf16(v[4 * q + 2], v[4 * q + 3])};
        }
  } else {
    const uint16_t* Rt = g.R + tile * g.r_bs + (int64_t)(ib + l32) * g.ldr + jb + 4 * hi;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      u32x2_t rv[2][4];
#pragma unroll
      for (int tj = 0; tj < 2; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          rv[tj][q] = *reinterpret_cast<const u32x2_t*>(Rt + (int64_t)(32 * ti) * g.ldr + 32 * tj + 8 * q);
#pragma unroll
      for (int tj = 0; tj < 2; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = bf16_to_f32(half16(rv[tj][q][e >> 1], e & 1));
            const float v = acc[tj][ti][4 * q + e];
            if constexpr (MODE == kApply)
              y[e] = fmaf(g.beta, x, bf16_to_f32(pk_bf16(v, 0.f) & 0xffffu));  // bf16(B X) + a X
            else
              y[e] = fmaf(g.beta, x, g.alpha * v);  // c (A A^T) + b A
          }
          out[ti][tj][q] = u32x2_t{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
        }
    }
  }
  lds_barrier();  // every wave is done with the ring: its LDS becomes staging
  if (!write) return;

  // Stage the wave's 128 x 64 sub-block (128-byte rows, chunk ^ swz_o(row)),
  // then store it with 16-byte lanes, 8 rows x 128 bytes per instruction.
  lds_u8* const W = lds + wave * WSTAGE;
#pragma unroll
  for (int ti = 0; ti < 4; ++ti)
#pragma unroll
    for (int tj = 0; tj < 2; ++tj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 32 * ti + l32, ch = 4 * tj + q;
        *reinterpret_cast<lds_u32x2*>(W + r * 128 + ((ch ^ swz_o(r)) * 16) + hi * 8) = out[ti][tj][q];
      }
  uint16_t* Ct = g.C + tile * g.c_bs;
  wait_lgkm<0>();
  {
    const int sr = lane >> 3, sc = lane & 7;
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      const int r = 8 * n + sr;
      const u32x4_t v = *reinterpret_cast<lds_cu32x4*>(W + r * 128 + ((sc ^ swz_o(r)) * 16));
      *reinterpret_cast<u32x4_t*>(Ct + (int64_t)(ib + r) * g.ldc + jb + sc * 8) = v;
    }
  }
  if constexpr (MODE != kApply) {
    if (mirror) {
      // Mirror block C[j][i]: after the quad transpose, lane (a = l32/4,
      // k = l32%4) holds C^T[jt][it .. it + 3], jt = 32 tj + 8 q + 4 hi + k,
      // it = 32 ti + 4 a (wave-local); staged as 64 rows x 256 bytes.
      wait_lgkm<0>();  // this wave's staging reads are done
      const int k = lane & 3, a = l32 >> 2;
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const u32x2_t tv = quad_transpose(out[ti][tj][q], k);
            const int r = 32 * tj + 8 * q + 4 * hi + k, ch = 4 * ti + (a >> 1);
            *reinterpret_cast<lds_u32x2*>(W + r * 256 + ((ch ^ swz_m(r)) * 16) + (a & 1) * 8) = tv;
          }
      wait_lgkm<0>();
      const int sr = lane >> 4, sc = lane & 15;
#pragma unroll
      for (int n = 0; n < 16; ++n) {
        const int r = 4 * n + sr;
        const u32x4_t v = *reinterpret_cast<lds_cu32x4*>(W + r * 256 + ((sc ^ swz_m(r)) * 16));
        *reinterpret_cast<u32x4_t*>(Ct + (int64_t)(jb + r) * g.ldc + ib + sc * 8) = v;
      }
    }
  }
}

// NKC: K units known at compile time (16: K = 512, the tile_size 512 case;
// 0: K from the arguments).
template <int MODE, int NKC>
__global__ __launch_bounds__(NT, 2) void ns_duo_kernel(DuoArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
  const int P = g.M / BI;
  const int ncb = g.N / BJ;
  const int per_tile = (MODE == kApply) ? P * ncb : P * (P + 1);
  const int64_t total = g.ntiles * per_tile;
  const int wper = (int)(gridDim.x >> 3);
  const int64_t per_xcd = (total + 7) >> 3;
  const int64_t ibeg = (int64_t)(blockIdx.x & 7) * per_xcd;
  const int64_t iend = (ibeg + per_xcd < total) ? ibeg + per_xcd : total;
  for (int64_t item = ibeg + (blockIdx.x >> 3); item < iend; item += wper) {
    const int64_t tile = item / per_tile;
    const int q = (int)(item - tile * per_tile);
    int p, c;
    if constexpr (MODE == kApply) {
      p = q / ncb;
      c = q - p * ncb;
    } else {
      p = 0;  // row block p holds items p (p + 1) .. p (p + 1) + 2 p + 1
      while ((p + 1) * (p + 2) <= q) ++p;
      c = q - p * (p + 1);
    }
    duo_item<MODE, NKC>(g, (lds_u8*)lds, tile, p, c);
  }
}

// X0 = bf16(x * inv) in place, 8 elements per thread.
__global__ __launch_bounds__(NT) void ns_duo_scale_kernel(uint16_t* __restrict__ x,
                                                          const float* __restrict__ inv,
                                                          int64_t per_tile, int64_t ntiles) {
  const int64_t nvec = ntiles * per_tile / 8;
  for (int64_t v = (int64_t)blockIdx.x * NT + threadIdx.x; v < nvec; v += (int64_t)gridDim.x * NT) {
    u32x4_t* px = reinterpret_cast<u32x4_t*>(x) + v;
    *px = scale8(*px, inv[(v * 8) / per_tile]);
  }
}

// ---------------------------------------------------------------------------
// Dataflow variant: one persistent launch runs all `steps` iterations of a
// sub-batch. Tiles are grouped in windows of W tiles; the workgroups of one
// XCD claim a whole window from a global counter, so every item of a tile
// runs on one XCD and its intermediates (A, B, X) pass through that XCD's L2
// (and the memory-side cache) instead of HBM. Within an XCD, items are
// claimed in queue order
//   window k: for it < steps: for stage (GramA, GramB, Apply): for tile of k: for block
// and an item waits until its tile's progress counter shows every item of the
// previous stage done. Dependencies only point to earlier queue positions of
// the same XCD, whose workgroups are running, so the waits always end; each
// wait is bounded all the same (on overrun the kernel sets `err` and drains).
//
// Coherence: producer and consumer of a tile's data share the XCD's L2. A
// producer waits for its stores (vmcnt 0) before it increments the tile's
// counter with an agent-scope atomic; a consumer that sees the count
// invalidates its CU's L1 (buffer_inv sc0) before loading.
struct FlowArgs {
  uint16_t* x; uint16_t* y;   // X ping-pong (cnt x mp x np)
  uint16_t* A; uint16_t* B;   // per-tile A and B (cnt x mp x mp)
  int* prog;                  // [cnt] items done per tile
  int* qctr;                  // [16] items claimed per XCD
  int* gwin;                  // windows claimed
  int* err;                   // non-zero after a wait overran its bound
  int* wseq;                  // [16][nwin + 1] global window of each XCD window (-1: not yet)
  int64_t cnt;
  int mp, np, steps, W, nwin;
  float a, b, c;
};

constexpr int kEndWindow = -2;
constexpr int kSpinLimit = 1 << 22;  // polls (each ~0.1-1 us) before a wait gives up

HM_DEV int ld_acq(const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
HM_DEV int xcc_id() { return (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15); }  // HW_REG_XCC_ID

// Claims the next item of XCD xq's queue; the claimant of a window's first
// item takes the next global window and publishes it.
HM_DEV int flow_claim(const FlowArgs& f, int xq, int ipw) {
  const int q = __hip_atomic_fetch_add(&f.qctr[xq], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int k = q / ipw;
  if (q % ipw == 0 && k < f.nwin) {
    const int g = __hip_atomic_fetch_add(f.gwin, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&f.wseq[xq * (f.nwin + 1) + k], g < f.nwin ? g : kEndWindow, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  return q;
}

// NKC: K units known at compile time (16: mp = np = 512; 0: from the shapes).
template <int NKC>
__global__ __launch_bounds__(NT, 2) void ns_flow_kernel(FlowArgs f) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
  __shared__ int s_next, s_tile, s_it, s_stage, s_blk;
  const int xq = xcc_id();
  const int P = f.mp / BI, ncb = f.np / BJ;
  const int ga = P * (P + 1), ap = P * ncb, ipt = 2 * ga + ap;  // items per tile-iteration
  const int ipw = f.W * f.steps * ipt;                           // items per full window
  const int64_t sq = (int64_t)f.mp * f.mp, rect = (int64_t)f.mp * f.np;
  if (threadIdx.x == 0) s_next = flow_claim(f, xq, ipw);
  __syncthreads();
  for (;;) {
    if (threadIdx.x == 0) {
      const int q = s_next;
      const int k = q / ipw, r = q - k * ipw;
      int tile = -1, it = 0, stage = 0, blk = 0;  // tile -1: end; -2: empty slot of a short window
      int g = kEndWindow;
      if (k < f.nwin) {
        int spins = 0;
        while ((g = ld_acq(&f.wseq[xq * (f.nwin + 1) + k])) == -1) {
          __builtin_amdgcn_s_sleep(2);
          if (++spins > kSpinLimit) { atomicOr(f.err, 1); g = kEndWindow; break; }
        }
      }
      if (g >= 0) {
        const int t0 = g * f.W;
        const int wsz = (int)min<int64_t>(f.W, f.cnt - t0);
        const int per_it = ipt * wsz;
        if (r >= f.steps * per_it) {
          tile = -2;
        } else {
          it = r / per_it;
          int r2 = r - it * per_it;
          if (r2 < ga * wsz) {
            stage = kGramA; tile = t0 + r2 / ga; blk = r2 % ga;
          } else if ((r2 -= ga * wsz) < ga * wsz) {
            stage = kGramB; tile = t0 + r2 / ga; blk = r2 % ga;
          } else {
            r2 -= ga * wsz;
            stage = kApply; tile = t0 + r2 / ap; blk = r2 % ap;
          }
          const int need = it * ipt + (stage == kGramA ? 0 : stage == kGramB ? ga : 2 * ga);
          int spins = 0;
          while (ld_acq(&f.prog[tile]) < need) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins > kSpinLimit) { atomicOr(f.err, 2); tile = -1; break; }
          }
        }
      }
      s_tile = tile; s_it = it; s_stage = stage; s_blk = blk;
      if (tile != -1) s_next = flow_claim(f, xq, ipw);
    }
    __syncthreads();
    const int tile = s_tile, it = s_it, stage = s_stage, blk = s_blk;
    __syncthreads();  // every wave has read the item before thread 0 writes the next
    if (tile == -1) break;
    if (tile < 0) continue;
    asm volatile("buffer_inv sc0" ::: "memory");  // drop stale L1 lines of this tile's data
    uint16_t* cur = (it & 1) ? f.y : f.x;
    uint16_t* nxt = (it & 1) ? f.x : f.y;
    if (stage == kApply) {
      const int p = blk / ncb, c = blk - (blk / ncb) * ncb;
      const DuoArgs ap_{f.B, sq, f.mp, cur, rect, f.np, cur, rect, f.np, nxt, rect, f.np,
                        f.mp, f.np, f.mp, f.cnt, 1.0f, f.a};
      duo_item<kApply, NKC>(ap_, (lds_u8*)lds, tile, p, c);
    } else {
      int p = 0;
      while ((p + 1) * (p + 2) <= blk) ++p;
      const int c = blk - p * (p + 1);
      if (stage == kGramA) {
        const DuoArgs ga_{cur, rect, f.np, cur, rect, f.np, nullptr, 0, 0, f.A, sq, f.mp,
                          f.mp, f.mp, f.np, f.cnt, 1.0f, 0.0f};
        duo_item<kGramA, NKC>(ga_, (lds_u8*)lds, tile, p, c);
      } else {
        const DuoArgs gb_{f.A, sq, f.mp, f.A, sq, f.mp, f.A, sq, f.mp, f.B, sq, f.mp,
                          f.mp, f.mp, f.mp, f.cnt, f.c, f.b};
        duo_item<kGramB, NKC>(gb_, (lds_u8*)lds, tile, p, c);
      }
    }
    wait_vm<0>();  // this wave's stores have reached the L2
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(&f.prog[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Resets the dataflow counters: prog, qctr, gwin, err to 0 and wseq to -1.
__global__ __launch_bounds__(NT) void ns_flow_reset_kernel(int* ctr, int64_t n_zero, int64_t n_neg) {
  for (int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x; i < n_zero + n_neg; i += (int64_t)gridDim.x * NT)
    ctr[i] = i < n_zero ? 0 : -1;
}

int g_num_cus[16] = {0};

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  const int d = dev & 15;
  if (g_num_cus[d] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_num_cus[d] = n;
  }
  return g_num_cus[d];
}

template <int MODE>
void launch(const DuoArgs& a, int64_t items, hipStream_t s) {
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t wgs_per_xcd = std::max<int64_t>(1, std::min<int64_t>(2 * num_cus() / 8, per_xcd));
  const dim3 grid((unsigned)(8 * wgs_per_xcd));
  if (a.K == 16 * BK)
    hipLaunchKernelGGL((ns_duo_kernel<MODE, 16>), grid, dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL((ns_duo_kernel<MODE, 0>), grid, dim3(NT), 0, s, a);
}

}  // namespace

bool ns5_duo_supported(int mp, int np) { return mp % BI == 0 && np % BJ == 0; }

// One sub-batch of `cnt` tiles, `steps` >= 1 iterations, ping-ponging X
// between x and y (x is scaled in place first); A and B live in the
// workspace.
void ns5_duo_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                 float a, float b, float c, uint16_t* wsA, uint16_t* wsB, hipStream_t s) {
  const int64_t sq = (int64_t)mp * mp, rect = (int64_t)mp * np;
  const int P = mp / BI;
  const int64_t gram_items = cnt * (int64_t)(P * (P + 1));
  const int64_t apply_items = cnt * (int64_t)P * (np / BJ);
  const int64_t nvec = cnt * rect / 8;
  hipLaunchKernelGGL(ns_duo_scale_kernel, dim3((unsigned)std::min<int64_t>((nvec + NT - 1) / NT, 65536)),
                     dim3(NT), 0, s, x, inv, rect, cnt);
  uint16_t* cur = x;
  uint16_t* nxt = y;
  for (int it = 0; it < steps; ++it) {
    const DuoArgs ga{cur, rect, np, cur, rect, np, nullptr, 0, 0, wsA, sq, mp, mp, mp, np, cnt, 1.0f, 0.0f};
    launch<kGramA>(ga, gram_items, s);
    const DuoArgs gb{wsA, sq, mp, wsA, sq, mp, wsA, sq, mp, wsB, sq, mp, mp, mp, mp, cnt, c, b};
    launch<kGramB>(gb, gram_items, s);
    const DuoArgs ap{wsB, sq, mp, cur, rect, np, cur, rect, np, nxt, rect, np, mp, np, mp, cnt, 1.0f, a};
    launch<kApply>(ap, apply_items, s);
    std::swap(cur, nxt);
  }
}

// Dataflow counters in the workspace tail: prog[cnt], qctr[16], gwin, err
// (padded to 32 ints), then wseq[16][cnt + 1] (sized for windows of one tile).
size_t ns5_flow_counter_bytes(int64_t cnt) {
  return (size_t)4 * ((size_t)cnt + 32 + 16 * ((size_t)cnt + 1));
}

void ns5_flow_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                  float a, float b, float c, uint16_t* wsA, uint16_t* wsB, int* counters, int window,
                  hipStream_t s) {
  const int64_t rect = (int64_t)mp * np;
  const int64_t nvec = cnt * rect / 8;
  hipLaunchKernelGGL(ns_duo_scale_kernel, dim3((unsigned)std::min<int64_t>((nvec + NT - 1) / NT, 65536)),
                     dim3(NT), 0, s, x, inv, rect, cnt);
  const int W = std::max(1, window);
  const int nwin = (int)((cnt + W - 1) / W);
  int* prog = counters;
  int* qctr = prog + cnt;
  int* gwin = qctr + 16;
  int* err = gwin + 1;
  int* wseq = qctr + 32;
  const int64_t n_zero = cnt + 32, n_neg = 16 * ((int64_t)nwin + 1);
  hipLaunchKernelGGL(ns_flow_reset_kernel, dim3((unsigned)std::min<int64_t>((n_zero + n_neg + NT - 1) / NT, 1024)),
                     dim3(NT), 0, s, counters, n_zero, n_neg);
  const FlowArgs f{x, y, wsA, wsB, prog, qctr, gwin, err, wseq, cnt, mp, np, steps, W, nwin, a, b, c};
  if (mp == 16 * BK && np == 16 * BK)
    hipLaunchKernelGGL(ns_flow_kernel<16>, dim3((unsigned)(2 * num_cus())), dim3(NT), 0, s, f);
  else
    hipLaunchKernelGGL(ns_flow_kernel<0>, dim3((unsigned)(2 * num_cus())), dim3(NT), 0, s, f);
}
