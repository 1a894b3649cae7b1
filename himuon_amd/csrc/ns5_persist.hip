// Persistent 256x256-block kernels for the three NS5 stages (NS tiles whose
// padded edges are multiples of 256), X kept in one orientation only.
//
//   GramA : C = A = bf16(X X^T)            P = Q = X (rows, K = n)   lower blocks + mirror
//   GramB : C = B = bf16(c A A^T + b A)    P = Q = A (rows, K = m)   lower blocks + mirror
//   Apply : C = X' = bf16(bf16(B X) + a X) P = B (rows, K = m), X read as [k][j]
// (ns5_smem.py:89-101, XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88).
//
// Per block, K streams in 64-wide slabs straight from global memory into LDS
// (global_load_lds_dwordx4, two stages: slab kt + 1 lands while slab kt is
// multiplied). The destination of a direct load is fixed (lane l writes bytes
// 16l..16l+15 of the wave's 1 KiB), so bank-conflict avoidance is done by
// choosing which 16-byte source chunk each lane fetches:
//  * row panels (P, and Q of the Gram stages): 256 rows x 128 B, chunk c of
//    row r stored at position c ^ (r & 7);
//  * the Apply's X panel: 64 k-rows x 512 B (256 columns), chunk c of row r
//    at c ^ s(r), s(r) = 10 (r & 1) + 4 ((r >> 1) & 1). Its MFMA operand (8
//    consecutive k of one column per lane) comes from two ds_read_b64_tr_b16
//    per fragment: within 16 lanes, lane 4a+b receives element b of the 8-byte
//    rows addressed by lanes a, a+4, a+8, a+12.
// 4 waves in 2x2, each a 128x128 sub-block of 4x4 v_mfma_f32_32x32x16_bf16
// tiles with swapped operands, so lane l holds C[row l%32][4 consecutive
// columns]. The epilogue converts to bf16 with v_cvt_pk_bf16_f32 (RNE) and
// stores 8-byte row segments; off-diagonal Gram blocks also store the mirror
// block from a 4x4 transpose across each lane quad (two DPP exchanges).
#include "ns5_kernels.h"

namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) const u32x4_t lds_u32x4;
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
typedef __attribute__((address_space(1))) const void gbl_void;

constexpr int NT = 256;
constexpr int BT = 256;                 // output block edge
constexpr int BK = 64;                  // K slab (elements)
constexpr int PANEL = BT * BK * 2;      // one operand slab: 32 KiB
constexpr int QBASE = 2 * PANEL;        // P stages at [0, 64K), Q stages at [64K, 128K)
constexpr int LDS_BYTES = 4 * PANEL;

enum { kGramA = 0, kGramB = 1, kApply = 2 };

struct PkArgs {
  const uint16_t* P; int64_t p_bs; int ldp;    // rows i (output rows), k-contiguous
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

// s_waitcnt vmcnt(0) / lgkmcnt(0), the other counters at their maxima.
HM_DEV void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
HM_DEV void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

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

// One 256x256 output block: C[tile][bi-block][bj-block]. Inlined into the
// kernel: out of line, the arguments arrive through a generic pointer and
// every global access becomes a FLAT instruction (which also counts in
// lgkmcnt, serialising the LDS waits).
template <int MODE>
__device__ __forceinline__ void pk_item(const PkArgs& g, lds_u8* lds, int64_t tile, int bi, int bj) {
  constexpr bool kTr = MODE == kApply;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  const int nk = g.K / BK;

  // ---- loaders ---------------------------------------------------------
  // Row panels: load i of wave w fills rows 32i + 8w .. +7; lane l lands at
  // row 32i + 8w + l/8, position l%8, so it reads chunk (l%8) ^ (l/8).
  const int lr = lane >> 3, lc = (lane & 7) ^ lr;
  const uint16_t* psrc = g.P + tile * g.p_bs + (int64_t)(bi * BT + 8 * wave + lr) * g.ldp + lc * 8;
  const int64_t pstep = 32 * (int64_t)g.ldp;
  const uint16_t* qsrc;
  int64_t qstep;
  if constexpr (kTr) {
    // X panel: load i of wave w fills k-rows 2(4i + w), +1; lane l lands at
    // row 2(4i + w) + l/32, position l%32, so it reads chunk (l%32) ^ s(row)
    // with s(row) = 10 (l/32) + 4 (w & 1).
    const int xr = 2 * wave + hi, xc = l32 ^ (10 * hi + 4 * (wave & 1));
    qsrc = g.Q + tile * g.q_bs + (int64_t)xr * g.ldq + bj * BT + xc * 8;
    qstep = 8 * (int64_t)g.ldq;
  } else {
    qsrc = g.Q + tile * g.q_bs + (int64_t)(bj * BT + 8 * wave + lr) * g.ldq + lc * 8;
    qstep = 32 * (int64_t)g.ldq;
  }
  lds_u8* const wdst = lds + wave * 1024;
  auto issue = [&](int kt, int st) {
    lds_u8* dp = wdst + st * PANEL;
    lds_u8* dq = wdst + QBASE + st * PANEL;
    const int64_t qk = kTr ? (int64_t)kt * BK * g.ldq : (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_global_load_lds((gbl_void*)(psrc + i * pstep + kt * BK), dp + i * 4096, 16, 0, 0);
      __builtin_amdgcn_global_load_lds((gbl_void*)(qsrc + i * qstep + qk), dq + i * 4096, 16, 0, 0);
    }
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  // ---- MFMA fragments of sub-step ks ------------------------------------
  // B operand (rows i of P): row l32 of a 32-row fragment, k-chunk 2 ks + hi
  // at position (2 ks + hi) ^ (l32 & 7). A operand (rows j): the same from Q
  // for the Gram stages; two transposing reads of the X panel for Apply.
  const int prow = (wm * 128 + l32) * 128, qrow = (wn * 128 + l32) * 128;
  const int r16 = lane & 15, te = r16 >> 2;
  const int tr_s = 10 * (te & 1) + 4 * (te >> 1);
  const int tr_row = 8 * hi + te;                                  // + 16 ks (+ 4)
  const int tr_chunk = wn * 16 + 2 * ((lane >> 4) & 1) + ((r16 & 3) >> 1);  // + 4 t
  const int tr_sub = (r16 & 1) * 8;
  auto frags = [&](int st, int ks, u32x4_t(&fa)[4], u32x4_t(&fb)[4]) {
    const lds_u8* ps = lds + st * PANEL;
    const lds_u8* qs = lds + QBASE + st * PANEL;
    const int pos = ((2 * ks + hi) ^ (l32 & 7)) * 16;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      fb[t] = *reinterpret_cast<lds_u32x4*>(ps + prow + t * 4096 + pos);
      if constexpr (kTr) {
        const int off = (16 * ks + tr_row) * 512 + (((tr_chunk + 4 * t) ^ tr_s) * 16) + tr_sub;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(qs + off));
        const i16x4_t up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(qs + off + 4 * 512));
        const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), u2 = __builtin_bit_cast(u32x2_t, up);
        fa[t] = u32x4_t{l2[0], l2[1], u2[0], u2[1]};
      } else {
        fa[t] = *reinterpret_cast<lds_u32x4*>(qs + qrow + t * 4096 + pos);
      }
    }
  };

  // One slab from stage st: sub-step ks + 1's fragment reads are issued ahead
  // of sub-step ks's 16 MFMAs (sched_barrier fences keep the scheduler from
  // sinking each read next to its MFMA and waiting on it); with LOAD, slab
  // ktn's 16 direct loads into the other stage are interleaved one per MFMA
  // of the first sub-step.
  constexpr int kMfma = 0x008, kVmem = 0x010;
  auto slab = [&](auto load_tag, int st, int ktn) {
    constexpr bool LOAD = decltype(load_tag)::value;
    u32x4_t fa[2][4], fb[2][4];
    frags(st, 0, fa[0], fb[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      // Sub-step ks's reads have landed (they had the previous 16 MFMAs to do
      // so). Waiting here keeps at most one sub-step of LDS reads in flight:
      // past the 15 the lgkmcnt field counts, the compiler waits for all.
      wait_lgkm0();
      if (ks + 1 < BK / 16) frags(st, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      if (LOAD && ks == 0) issue(ktn, st ^ 1);
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
          acc[tj][ti] = mfma(fa[ks & 1][tj], fb[ks & 1][ti], acc[tj][ti]);
      if (LOAD && ks == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kVmem, 1, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using kLoad = std::integral_constant<bool, true>;
  using kNoLoad = std::integral_constant<bool, false>;

  // Slab kt + 1 loads into the other stage while slab kt is multiplied; the
  // barrier after each wave's vmcnt(0) publishes slab kt to every wave and
  // tells the loader that slab kt - 1's stage is free again. nk is even (K is
  // a multiple of 256) and the last pair is peeled, so the MFMAs sit in
  // straight-line code: a conditional around them makes the register
  // allocator shuttle the accumulators between AGPRs and VGPRs.
  __syncthreads();  // the previous item's last reads of the stage buffers are done
  issue(0, 0);
  wait_vm0();
  __syncthreads();
  for (int kt = 0; kt < nk - 2; kt += 2) {
    slab(kLoad{}, 0, kt + 1);
    wait_vm0();
    __syncthreads();
    slab(kLoad{}, 1, kt + 2);
    wait_vm0();
    __syncthreads();
  }
  slab(kLoad{}, 0, nk - 1);
  wait_vm0();
  __syncthreads();
  // The epilogue operand R (A or X) loads in the shadow of the last slab.
  u32x2_t out[4][4][4];
  const int i0 = bi * BT + wm * 128 + l32, j0 = bj * BT + wn * 128 + 4 * hi;
  if constexpr (MODE != kGramA) {
    const uint16_t* rb = g.R + tile * g.r_bs;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          out[ti][tj][q] =
              *reinterpret_cast<const u32x2_t*>(rb + (int64_t)(i0 + ti * 32) * g.ldr + j0 + tj * 32 + 8 * q);
  }
  slab(kNoLoad{}, 1, 0);

  // ---- epilogue: lane holds C[i0 + 32 ti][j0 + 32 tj + 8 q + e] ---------
#pragma unroll
  for (int ti = 0; ti < 4; ++ti)
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[tj][ti][4 * q + e];
        if constexpr (MODE == kGramA) {
          out[ti][tj][q][0] = pk_bf16(v[0], v[1]);
          out[ti][tj][q][1] = pk_bf16(v[2], v[3]);
        } else {
          const u32x2_t rv = out[ti][tj][q];
          float x[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = bf16_to_f32(half16(rv[e >> 1], e & 1));
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (MODE == kApply) {
              const uint32_t pr = pk_bf16(v[e], 0.f);  // bf16(B X)
              y[e] = fmaf(g.beta, x[e], bf16_to_f32(pr & 0xffffu));
            } else {
              y[e] = fmaf(g.beta, x[e], g.alpha * v[e]);
            }
          }
          out[ti][tj][q][0] = pk_bf16(y[0], y[1]);
          out[ti][tj][q][1] = pk_bf16(y[2], y[3]);
        }
      }
  uint16_t* Ct = g.C + tile * g.c_bs;
#pragma unroll
  for (int ti = 0; ti < 4; ++ti)
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<u32x2_t*>(Ct + (int64_t)(i0 + ti * 32) * g.ldc + j0 + tj * 32 + 8 * q) =
            out[ti][tj][q];
  if (MODE != kApply && bi != bj) {
    // Mirror block: lane k of each quad holds C^T[j + k][i..i+3] after the
    // quad transpose, i = i0 + 32 ti - (l32 & 3), j = j0 + 32 tj + 8 q.
    const int k = lane & 3;
    const int mi = i0 - k;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x2_t tv = quad_transpose(out[ti][tj][q], k);
          *reinterpret_cast<u32x2_t*>(Ct + (int64_t)(j0 + tj * 32 + 8 * q + k) * g.ldc + mi + ti * 32) = tv;
        }
  }
}

template <int MODE>
__global__ __launch_bounds__(NT, 1) void ns_pk_kernel(PkArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
  const int nbi = g.M / BT, nbj = g.N / BT;
  const int per_tile = (MODE == kApply) ? nbi * nbj : nbi * (nbi + 1) / 2;
  const int64_t total = g.ntiles * per_tile;
  const int wper = (int)(gridDim.x >> 3);
  const int64_t per_xcd = (total + 7) >> 3;
  const int64_t ibeg = (int64_t)(blockIdx.x & 7) * per_xcd;
  const int64_t iend = (ibeg + per_xcd < total) ? ibeg + per_xcd : total;
  for (int64_t item = ibeg + (blockIdx.x >> 3); item < iend; item += wper) {
    const int64_t tile = item / per_tile;
    const int p = (int)(item - tile * per_tile);
    int bi, bj;
    if (MODE == kApply) {
      bi = p / nbj;
      bj = p - bi * nbj;
    } else {
      bi = 0;
      while ((bi + 1) * (bi + 2) / 2 <= p) ++bi;
      bj = p - bi * (bi + 1) / 2;
    }
    pk_item<MODE>(g, (lds_u8*)lds, tile, bi, bj);
  }
}

// X0 = bf16(x * inv) in place, 8 elements per thread.
__global__ __launch_bounds__(NT) void ns_pk_scale_kernel(uint16_t* __restrict__ x,
                                                         const float* __restrict__ inv,
                                                         int64_t per_tile, int64_t ntiles) {
  const int64_t nvec = ntiles * per_tile / 8;
  for (int64_t v = (int64_t)blockIdx.x * NT + threadIdx.x; v < nvec; v += (int64_t)gridDim.x * NT) {
    u32x4_t* p = reinterpret_cast<u32x4_t*>(x) + v;
    *p = scale8(*p, inv[(v * 8) / per_tile]);
  }
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
void launch(const PkArgs& a, int64_t items, hipStream_t s) {
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t wgs_per_xcd = std::max<int64_t>(1, std::min<int64_t>(num_cus() / 8, per_xcd));
  hipLaunchKernelGGL((ns_pk_kernel<MODE>), dim3((unsigned)(8 * wgs_per_xcd)), dim3(NT), 0, s, a);
}

}  // namespace

bool ns5_pk_supported(int mp, int np) { return mp % BT == 0 && np % BT == 0; }

// One sub-batch of `cnt` tiles, `steps` >= 1 iterations, ping-ponging X
// between x and y (x is scaled in place first); A and B live in the
// workspace.
void ns5_pk_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                float a, float b, float c, uint16_t* wsA, uint16_t* wsB, hipStream_t s) {
  const int64_t sq = (int64_t)mp * mp, rect = (int64_t)mp * np;
  const int nb = mp / BT;
  const int64_t gram_items = cnt * (nb * (nb + 1) / 2);
  const int64_t apply_items = cnt * nb * (np / BT);
  const int64_t nvec = cnt * rect / 8;
  hipLaunchKernelGGL(ns_pk_scale_kernel, dim3((unsigned)std::min<int64_t>((nvec + NT - 1) / NT, 65536)),
                     dim3(NT), 0, s, x, inv, rect, cnt);
  uint16_t* cur = x;
  uint16_t* nxt = y;
  for (int it = 0; it < steps; ++it) {
    const PkArgs ga{cur, rect, np, cur, rect, np, nullptr, 0, 0, wsA, sq, mp, mp, mp, np, cnt, 1.0f, 0.0f};
    launch<kGramA>(ga, gram_items, s);
    const PkArgs gb{wsA, sq, mp, wsA, sq, mp, wsA, sq, mp, wsB, sq, mp, mp, mp, mp, cnt, c, b};
    launch<kGramB>(gb, gram_items, s);
    const PkArgs ap{wsB, sq, mp, cur, rect, np, cur, rect, np, nxt, rect, np, mp, np, mp, cnt, 1.0f, a};
    launch<kApply>(ap, apply_items, s);
    std::swap(cur, nxt);
  }
}
