// Persistent streamed-operand kernels for the three NS5 stages on 256x256
// output blocks (NS tiles whose padded edges are multiples of 256):
//
//   GramA : C = A = bf16(X X^T)            P = Q = X (rows, K = n)   lower blocks + mirror
//   GramB : C = B = bf16(c A A^T + b A)    P = Q = A (rows, K = m)   lower blocks + mirror
//   Apply : C = X' = bf16(bf16(B X) + a X) P = B (rows, K = m), Q = X read as [k][j]
// (ns5_smem.py:89-101, XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88).
//
// One workgroup per CU walks a contiguous range of output blocks of its XCD:
// 8 waves in 2x4, two per SIMD, each a 128x64 sub-block of 4x2
// v_mfma_f32_32x32x16_bf16 tiles (128 fp32 accumulators per lane), so that
// one wave's MFMAs run while the other on its SIMD waits at a barrier or
// issues loads. (The code also takes 4 waves in 2x2 of 128x128 each, one
// per SIMD; that layout measured slower.)
//
// Operand stream. K advances in units of 32. Each unit of P (and Q) goes
// straight from global memory into a 32 KiB slot of a 5-slot LDS ring
// (global_load_lds_dwordx4, 1 KiB per wave instruction); loads run 4 units
// ahead of the MFMAs, so up to 128 KiB per CU are in flight (GramA: 4 slots,
// 3 units ahead). The epilogue
// operand R (A for GramB, X for Apply) is streamed behind the last K unit as
// four more 32 KiB units (64 rows x 256 columns each), so it lands while the
// last MFMAs run. A direct load writes lane l's 16 bytes at 16 l of the wave's
// 1 KiB, so LDS bank spreading is done by choosing which 16-byte source chunk
// each lane fetches (a per-row XOR swizzle of the chunk index).
//
// MFMA operands are swapped (A operand = rows j, B operand = rows i), so lane
// l holds C[row l%32][4 consecutive columns]. The epilogue converts in
// registers, then first issues the workgroup's next item's first 4 K units
// into ring slots 0..3, so that their latency, and the drain of this item's
// stores (vmcnt retires loads and stores in issue order), overlap this
// epilogue instead of stalling the next item's start. It then stages each
// wave's 128x128 bf16 result through its 8 KiB quarter of ring slot 4, in 4
// rounds of 32 rows, and writes it with 16-byte row-contiguous stores (256
// bytes per row). Off-diagonal Gram blocks also write the mirrored block: a
// 4x4 transpose across each lane quad (two DPP exchanges) restages the
// sub-block as rows of C^T.
#include "ns5_kernels.h"

namespace {


typedef __attribute__((address_space(3))) u32x4_t lds_u32x4;

constexpr int BT = 256;               // output block edge
constexpr int BK = 32;                // K per stream unit
constexpr int SLOT = 32768;           // bytes per ring slot
constexpr int HALF = SLOT / 2;        // Q panel offset within a slot

enum { kGramA = 0, kGramB = 1, kApply = 2 };

// Ring slots; units in flight ahead of the MFMAs = slots - 1. GramB and
// Apply stream their epilogue operand R as four units behind the K loop
// and take 5 slots; GramA has no R, and 4 slots are 1-3 % faster there.
template <int MODE>
constexpr int kSlots = MODE == kGramA ? 4 : 5;

struct StArgs {
  const uint16_t* P; int64_t p_bs; int ldp;    // rows i (output rows), k-contiguous
  const uint16_t* Q; int64_t q_bs; int ldq;    // Gram: rows j, k-contiguous; Apply: X [k][j]
  const uint16_t* R; int64_t r_bs; int ldr;    // epilogue operand [i][j] (A or X)
  uint16_t* C; int64_t c_bs; int ldc;          // output [i][j]
  int M, N, K;
  int64_t ntiles;
  float alpha, beta;                           // GramB: c, b; Apply: beta = a
  int round_once;                              // Apply: bf16(B X + a X), one rounding
  const float* inv;                            // SC kernels: X0 = bf16(X inv[tile]) on load
};

// Chunk swizzles (16-byte chunk index XOR a function of the row):
//  P/Q row panels, 64-byte rows: spreads 8 (or 16) consecutive rows of one
//  chunk over distinct bank groups for 32- and 64-bank layouts;
//  X panel of Apply, 512-byte rows: the transposing reads of 4 rows x 32
//  bytes hit distinct bank groups;
//  R units and the output staging, 512/256-byte rows: consecutive rows of
//  one chunk land in distinct bank groups.
HM_DEV int swz_p(int r) { return (((r >> 1) ^ (r >> 3)) & 1) | (((r >> 2) & 1) << 1); }
HM_DEV int swz_x(int r) { return 10 * (r & 1) + 4 * ((r >> 1) & 1); }
HM_DEV int swz_c(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// vmcnt while waiting for unit w, with DI units in flight: the loads of the
// (up to DI - 1) units issued after it (a K unit is L loads per wave, an R
// unit RL; with rem K units left after w, the rest of the DI - 1 are R units,
// at most NR) and, when this item's first DI units were prefetched during the
// previous item's epilogue, the sp global stores of that epilogue, which were
// issued after unit DI - 1 and before unit DI (vmcnt counts loads and stores
// together and retires them in issue order). sp is 0, 16, 32 or 64; with 64
// the count is capped at the counter's maximum, which waits for slightly more
// than needed.
template <int L, int NR, int RL, int DI>
HM_DEV void wait_unit(int nk, int w, int sp) {
  constexpr auto rmin = [](int a, int b) { return a < b ? a : b; };
  const int rem = nk - 1 - w;
  if (w < DI && sp > 0) {  // nk >= 8, so rem >= DI here; sp is 16, 32 or 64
    if (sp > 32)
      wait_vm<63>();
    else if (sp == 16)
      wait_vm<(DI - 1) * L + 16>();
    else
      wait_vm<(DI - 1) * L + 32>();
  } else if (rem >= DI - 1) {
    wait_vm<(DI - 1) * L>();
  } else if (rem == 2) {
    wait_vm<2 * L + RL * rmin(NR, DI - 3)>();
  } else if (rem == 1) {
    wait_vm<L + RL * rmin(NR, DI - 2)>();
  } else {
    wait_vm<RL * rmin(NR, DI - 1)>();
  }
}

// Item position: output block (bi, bj) of one tile.
struct ItemPos {
  int64_t tile;
  int bi, bj;
  bool diag;  // Gram diagonal block (Q = P, no mirror)
};

// Per-lane global sources of an item's P and Q operand units.
struct ItemSrc {
  const uint16_t* p;
  const uint16_t* q;
  int64_t pstep, qstep, qunit;
};

// NW waves per workgroup share each unit's 32 one-KiB load instructions.
template <int MODE, int NW>
HM_DEV ItemSrc item_src(const StArgs& g, const ItemPos& it, int lane, int wave) {
  // Row panel (256 rows x 64 B): wave instruction n = NW i + wave fills rows
  // 16 n .. 16 n + 15; lane l lands at row 16 n + l/4, position l%4 and
  // fetches chunk (l%4) ^ swz_p(row) (row & 15 = l/4).
  const int prl = lane >> 2;
  const int pch = (lane & 3) ^ swz_p(prl);
  ItemSrc s;
  s.p = g.P + it.tile * g.p_bs + (int64_t)(it.bi * BT + 16 * wave + prl) * g.ldp + pch * 8;
  s.pstep = 16 * NW * (int64_t)g.ldp;
  if constexpr (MODE == kApply) {
    // X panel (32 k-rows x 512 B): instruction n fills k-rows 2n, 2n + 1;
    // lane l lands at row 2n + l/32, position l%32, fetching chunk
    // (l%32) ^ swz_x(row) (row & 3 = (2 wave + hi) & 3).
    const int xr = 2 * wave + (lane >> 5);
    const int xc = (lane & 31) ^ swz_x(xr);
    s.q = g.Q + it.tile * g.q_bs + (int64_t)xr * g.ldq + it.bj * BT + xc * 8;
    s.qstep = 2 * NW * (int64_t)g.ldq;
    s.qunit = BK * (int64_t)g.ldq;
  } else {
    s.q = g.Q + it.tile * g.q_bs + (int64_t)(it.bj * BT + 16 * wave + prl) * g.ldq + pch * 8;
    s.qstep = 16 * NW * (int64_t)g.ldq;
    s.qunit = BK;
  }
  return s;
}

// K unit v of an item into ring slot `slot` (wdst = the wave's 1 KiB part).
template <int NW>
HM_DEV void issue_k(const ItemSrc& s, uint32_t wdst, int v, int slot, bool diag) {
  const uint32_t d = wdst + slot * SLOT;
#pragma unroll
  for (int i = 0; i < 16 / NW; ++i)
    dma16(s.p + i * s.pstep + v * BK, d + i * NW * 1024);
  if (!diag) {
#pragma unroll
    for (int i = 0; i < 16 / NW; ++i)
      dma16(s.q + i * s.qstep + v * s.qunit, d + HALF + i * NW * 1024);
  }
}

// One 256x256 output block C[tile][bi-block][bj-block]. DIAG: Gram diagonal
// block, Q = P (one panel streamed), no mirror.
//
// pre_st: 0 if this item's first DIST units are still to be issued, else the
// number of global stores (32 or 64) the previous item's epilogue issued
// after prefetching them. nx: the next item of this workgroup (if `more`); its
// first DIST units are issued into ring slots 0..DIST-1 as soon as this
// item no longer needs the ring, before this item's stores, so that neither
// their latency nor the store drain is exposed at the next item's start.
// Returns the number of global stores issued by this item's epilogue.
//
// NW = 4: waves in 2 x 2, each a 128x128 sub-block (4x4 MFMA tiles, 256
// accumulators per lane, one wave per SIMD). NW = 8: waves in 2 x 4, each
// 128x64 (4x2 tiles, 128 accumulators, two waves per SIMD, so that one
// wave's MFMAs can run while the other waits or issues loads).
//
// SC (GramA and Apply of the first iteration): the X operand is the raw
// tile; every X value is replaced by bf16(x inv[tile]) as it enters the
// computation (fragments after their LDS reads, the Apply epilogue's a X
// term), which is X0 exactly as a separate scaling pass would write it.
template <int MODE, bool DIAG, int NKC, int NW, bool SC>
__device__ __forceinline__ int st_item(const StArgs& g, lds_u8* lds, const ItemPos it, int pre_st,
                                       const bool more, const ItemPos nx) {
  constexpr bool kTr = MODE == kApply;
  constexpr int NR = (MODE == kGramA) ? 0 : 4;   // R units
  constexpr int WN = NW / 2;                      // waves along the block's columns
  constexpr int WC = BT / WN;                     // columns per wave (128 or 64)
  constexpr int TJ = WC / 32;                     // MFMA tiles along a wave's columns
  constexpr int L = (DIAG ? 16 : 32) / NW;        // K-unit loads per wave
  constexpr int RL = 32 / NW;                     // R-unit loads per wave
  constexpr int NSLOT = kSlots<MODE>;             // ring slots
  constexpr int DIST = NSLOT - 1;                 // units in flight ahead of the MFMAs
  const int64_t tile = it.tile;
  const int bi = it.bi, bj = it.bj;
  // The lane index is made opaque per block so that the per-lane addresses
  // below are recomputed for each block instead of being hoisted out of the
  // persistent loop (where they would not fit in registers).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, hi = lane >> 5;
  const int nk = NKC > 0 ? NKC : g.K / BK;  // K units (compile-time for the common K)
  const int U = nk + NR;
  static_assert(!SC || MODE != kGramB, "GramB has no X operand");
  float xs = 1.f;
  if constexpr (SC) xs = uniform_load_f32(g.inv, tile);

  // ---- loaders ------------------------------------------------------------
  const ItemSrc src = item_src<MODE, NW>(g, it, lane, wave);
  // R unit q (block rows 64 q .. 64 q + 63, 256 columns, 512-byte rows):
  // instruction n = NW i + wave fills rows 2n, 2n + 1; chunk (l%32) ^ (row & 15).
  const uint16_t* rsrc = nullptr;
  if constexpr (NR > 0)
    rsrc = g.R + tile * g.r_bs + (int64_t)(bi * BT + 2 * wave + hi) * g.ldr + bj * BT;
  const uint32_t wdst = (uint32_t)(uintptr_t)lds + wave * 1024;

  auto issue = [&](int v) {
    const int slot = v % NSLOT;
    if (v < nk) {
      issue_k<NW>(src, wdst, v, slot, DIAG);
    } else if constexpr (NR > 0) {
      const uint32_t d = wdst + slot * SLOT;
      const int q = v - nk;
#pragma unroll
      for (int i = 0; i < RL; ++i) {
        const int sw = (2 * NW * i + 2 * wave + hi) & 15;  // row & 15
        const uint16_t* s = rsrc + (int64_t)(64 * q + 2 * NW * i) * g.ldr + ((l32 ^ sw) * 8);
        dma16(s, d + i * NW * 1024);
      }
    }
  };

  // ---- MFMA fragments of unit v, sub-step ks --------------------------------
  // B operand (rows i = wm*128 + 32 t + l32 of P): k-chunk 2 ks + hi. A
  // operand: the same from Q (rows j) for Gram; for Apply two transposing
  // reads of the X panel (ds_read_b64_tr_b16: within 16 lanes, lane 4a+b
  // receives element b of the 8-byte rows addressed by lanes a, a+4, a+8,
  // a+12), giving lane l column j = wn*WC + 32 t + l%32, k = 16 ks + 8 hi + 0..7.
  const int sp = swz_p(l32 & 15);
  const int prow = (wm * 128 + l32) * 64, qrow = (wn * WC + l32) * 64;
  const int r16 = lane & 15, te = r16 >> 2;
  const int tr_s = swz_x(te);
  const int tr_row = 8 * hi + te;
  const int tr_chunk = wn * (WC / 8) + 2 * ((lane >> 4) & 1) + ((r16 & 3) >> 1);
  const uint32_t tr_lane = (uint32_t)(uintptr_t)lds + HALF + tr_row * 512 + (r16 & 1) * 8;
  // which: 1 = P fragments (fb), 2 = Q fragments (fa), 3 = both.
  auto frags = [&](int v, int ks, u32x4_t(&fa)[TJ], u32x4_t(&fb)[4], int which = 3) {
    const lds_u8* s = lds + (v % NSLOT) * SLOT;
    const int pos = ((2 * ks + hi) ^ sp) * 16;
    if (which & 1) {
#pragma unroll
      for (int t = 0; t < 4; ++t) fb[t] = *reinterpret_cast<lds_cu32x4*>(s + prow + t * 2048 + pos);
    }
    if (!(which & 2)) return;
    // Apply: the lane's read base is made opaque per call, so the addresses
    // of equal (slot, ks) in different units of the unrolled K loop are not
    // merged and kept live across units; rows 4 .. 7 of a read pair come from
    // the instruction's offset field.
    uint32_t trb = tr_lane;
    if constexpr (kTr) asm volatile("" : "+v"(trb));
    trb += (v % NSLOT) * SLOT + 16 * ks * 512;
#pragma unroll
    for (int t = 0; t < TJ; ++t) {
      if constexpr (kTr) {
        const uint32_t off = trb + (((tr_chunk + 4 * t) ^ tr_s) * 16);
        const u32x2_t l2 = ds_read_tr16(off), u2 = ds_read_tr16<4 * 512>(off);
        fa[t] = u32x4_t{l2[0], l2[1], u2[0], u2[1]};
      } else {
        const lds_u8* qs = DIAG ? s : s + HALF;
        fa[t] = *reinterpret_cast<lds_cu32x4*>(qs + qrow + t * 2048 + pos);
      }
    }
  };

  // X0 scaling (SC). Apply: the X fragments as they land, called right after
  // the lgkmcnt wait for them, before further LDS reads are issued; they come
  // from inline-assembly reads that the compiler does not track, so each
  // passes through a wait that names it as an operand and the scaling cannot
  // be scheduled before the data has landed.
  auto scale_frags = [&](u32x4_t(&fa)[TJ], u32x4_t(&fb)[4]) {
    (void)fb;
    if constexpr (SC && kTr) {
#pragma unroll
      for (int t = 0; t < TJ; ++t) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fa[t]));
#pragma unroll
      for (int t = 0; t < TJ; ++t) fa[t] = scale8_rne(fa[t], xs);
    }
  };
  // GramA: unit v in LDS, scaled in place once, each wave its own DMA'd
  // 16-byte pieces (lane l's at 16 l of each of the wave's 1 KiB blocks),
  // after its wait for them and before the barrier that publishes the unit:
  // a third of the work of scaling every fragment read (each unit's bytes
  // are read as fragments by three waves on average).
  auto scale_unit = [&](int v) {
    if constexpr (SC && MODE == kGramA) {
      asm volatile("" ::: "memory");  // the reads below follow the vmcnt wait
      lds_u8* const d = lds + (v % NSLOT) * SLOT + wave * 1024 + 16 * lane;
#pragma unroll
      for (int i = 0; i < 16 / NW; ++i) {
        lds_u32x4* const p = reinterpret_cast<lds_u32x4*>(d + i * NW * 1024);
        *p = scale8_rne(*p, xs);
        if constexpr (!DIAG) {
          lds_u32x4* const q = reinterpret_cast<lds_u32x4*>(d + HALF + i * NW * 1024);
          *q = scale8_rne(*q, xs);
        }
      }
    }
  };

  f32x16_t acc[TJ][4];
#pragma unroll
  for (int a = 0; a < TJ; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;
  auto mma = [&](const u32x4_t(&fa)[TJ], const u32x4_t(&fb)[4]) {
#pragma unroll
    for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
  };
  auto mma_row = [&](const u32x4_t(&fa)[TJ], const u32x4_t(&fb)[4], int tj) {
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
  };

  // ---- K loop ------------------------------------------------------------------
  // Unit u lives in slot u % NSLOT. At the top of unit u + 1 each wave waits
  // for its own loads of that unit, then the barrier publishes the unit and
  // frees slot u % NSLOT (every wave has its unit-u fragments in registers),
  // which receives unit u + 1 + DIST. The second half of unit u's MFMAs runs
  // after the barrier, covering the first fragment reads of unit u + 1.
  if (pre_st == 0) {
    lds_barrier();  // the previous block's epilogue is done with the LDS
#pragma unroll
    for (int v = 0; v < DIST; ++v) issue(v);
  }
  wait_unit<L, NR, RL, DIST>(nk, 0, pre_st);
  scale_unit(0);
  lds_barrier();  // unit 0 is in; every wave is past the previous epilogue's staging
  issue(DIST);
  u32x4_t fa0[TJ], fb0[4], fa1[TJ], fb1[4];
  // At most one half-unit of fragment reads is in flight at any time (8 or 12
  // LDS operations: lgkmcnt counts to 15). Unit u: the first-half fragments
  // have landed at its start and the second-half reads are in flight; each
  // half's reads are issued ahead of the other half's 16 MFMAs.
  frags(0, 0, fa0, fb0);
  wait_lgkm<0>();
  scale_frags(fa0, fb0);
  __builtin_amdgcn_sched_barrier(0);
  frags(0, 1, fa1, fb1);
  __builtin_amdgcn_sched_barrier(0);
  // After the barrier, the DMA issue of unit u + 1 + DIST and the first-half
  // fragment reads of unit u + 1 go between the rows of unit u's second-half
  // MFMAs, so that they issue while the MFMA pipe is busy.
  auto unit = [&](int u) {
    mma(fa0, fb0);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm<0>();  // second-half fragments of unit u
    scale_frags(fa1, fb1);
    wait_unit<L, NR, RL, DIST>(nk, u + 1, pre_st);
    scale_unit(u + 1);
    lds_barrier();
    mma_row(fa1, fb1, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (u + 1 + DIST < U) issue(u + 1 + DIST);
    __builtin_amdgcn_sched_barrier(0);
    mma_row(fa1, fb1, 1);
    __builtin_amdgcn_sched_barrier(0);
    frags(u + 1, 0, fa0, fb0, 1);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (TJ > 2) {
      mma_row(fa1, fb1, 2);
      __builtin_amdgcn_sched_barrier(0);
    }
    frags(u + 1, 0, fa0, fb0, 2);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (TJ > 3) mma_row(fa1, fb1, 3);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm<0>();  // first-half fragments of unit u + 1
    scale_frags(fa0, fb0);
    __builtin_amdgcn_sched_barrier(0);
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
  scale_frags(fa1, fb1);
  mma(fa1, fb1);

  // ---- epilogue ------------------------------------------------------------------
  // out[ti][tj][q] = 4 bf16 of C[i][j..j+3], i = wm*128 + 32 ti + l32,
  // j = wn*WC + 32 tj + 8 q + 4 hi (block-local).
  u32x2_t out[4][TJ][4];
  if constexpr (NR > 0) {
    wait_vm<0>();
    lds_barrier();  // every wave's R loads have landed
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int il = wm * 128 + 32 * ti + l32;
      const int rq = il & 63;
      const lds_u8* rs = lds + ((nk + (il >> 6)) % NSLOT) * SLOT + rq * 512 + hi * 8;
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int ch = wn * (WC / 8) + 4 * tj + q;
          const u32x2_t rv = *reinterpret_cast<lds_cu32x2*>(rs + ((ch ^ (rq & 15)) * 16));
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = bf16_to_f32(half16(rv[e >> 1], e & 1));
            if constexpr (SC) x = bf16_to_f32(pk_bf16(x * xs, 0.f) & 0xffffu);
            const float v = acc[tj][ti][4 * q + e];
            if constexpr (MODE == kApply)  // bf16(B X) + a X, or B X + a X (2-D form)
              y[e] = fmaf(g.beta, x, g.round_once ? v : bf16_to_f32(pk_bf16(v, 0.f) & 0xffffu));
            else
              y[e] = fmaf(g.beta, x, g.alpha * v);  // c (A A^T) + b A
          }
          out[ti][tj][q] = u32x2_t{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
        }
    }
  } else {
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x16_t& v = acc[tj][ti];
          out[ti][tj][q] = u32x2_t{pk_bf16(v[4 * q], v[4 * q + 1]), pk_bf16(v[4 * q + 2], v[4 * q + 3])};
        }
  }
  lds_barrier();  // all fragment and R reads are done: the ring is free

  // The next item's first DIST units go to ring slots 0..DIST-1 now, ahead
  // of this item's stores; slot DIST is the staging area.
  if (more) {
    const ItemSrc ns = item_src<MODE, NW>(g, nx, lane, wave);
#pragma unroll
    for (int v = 0; v < DIST; ++v) issue_k<NW>(ns, wdst, v, v, nx.diag);
  }

  // Output stores are non-temporal: the block is not read again by this
  // launch, and its lines should not displace operand rows other workgroups
  // of the XCD still stream from L2.
  // Staging in 4 rounds per block: each wave stages 32 rows x WC columns
  // (WC * 2-byte rows) in its 1/NW of slot DIST, then stores them with
  // 16-byte lanes, whole rows per instruction: 8 (NW = 4) or 4 (NW = 8)
  // stores per round. LDS operations of one wave execute in order, so a
  // round's writes may follow the previous round's reads without a wait.
  // Row swizzle: 256-byte rows chunk ^ swz_c(row); 128-byte rows (two per
  // 256-byte bank line) chunk ^ ((row >> 1) & 7).
  constexpr int RB = WC * 2, CPR = WC / 8, RPI = 64 / CPR;
  lds_u8* const W = lds + DIST * SLOT + wave * (SLOT / NW);
  auto swz_s = [](int r) { return CPR == 16 ? swz_c(r) : ((r >> 1) & 7); };
  uint16_t* Ct = g.C + tile * g.c_bs;
  uint16_t* const cdst = Ct + (int64_t)(bi * BT + wm * 128) * g.ldc + bj * BT + wn * WC;
  {
    const int srow = lane / CPR, sch = lane % CPR;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int ch = 4 * tj + q;
          *reinterpret_cast<lds_u32x2*>(W + l32 * RB + ((ch ^ swz_s(l32)) * 16) + hi * 8) = out[ti][tj][q];
        }
      uint16_t* const dst = cdst + (int64_t)(32 * ti) * g.ldc;
#pragma unroll
      for (int n = 0; n < 32 / RPI; ++n) {
        const int r = RPI * n + srow;
        const u32x4_t v = *reinterpret_cast<lds_cu32x4*>(W + r * RB + ((sch ^ swz_s(r)) * 16));
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(dst + (int64_t)r * g.ldc + sch * 8));
      }
    }
  }
  int stores = 4 * (32 / RPI);
  if constexpr (MODE != kApply && !DIAG) {
    // Mirror block (bj, bi): after the quad transpose, lane (a = l32/4,
    // k = l32%4) holds C^T[jt][it..it+3], jt = 32 tj + 8 q + 4 hi + k,
    // it = 32 ti + 4 a (wave-local): 256-byte rows. A round stages MR rows
    // (32 for NW = 4: all q of one tj; 16 for NW = 8: a pair of q).
    constexpr int MR = (SLOT / NW) / 256, QR = MR / 8;
    uint16_t* const mdst = Ct + (int64_t)(bj * BT + wn * WC) * g.ldc + bi * BT + wm * 128;
    const int k = lane & 3, a = l32 >> 2;
    const int srow = lane >> 4, sch = lane & 15;
#pragma unroll
    for (int tj = 0; tj < TJ; ++tj) {
#pragma unroll
      for (int q0 = 0; q0 < 4; q0 += QR) {
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
#pragma unroll
          for (int qq = 0; qq < QR; ++qq) {
            const u32x2_t tv = quad_transpose(out[ti][tj][q0 + qq], k);
            const int r = 8 * qq + 4 * hi + k, ch = 4 * ti + (a >> 1);
            *reinterpret_cast<lds_u32x2*>(W + r * 256 + ((ch ^ swz_c(r)) * 16) + (a & 1) * 8) = tv;
          }
        uint16_t* const dst = mdst + (int64_t)(32 * tj + 8 * q0) * g.ldc;
#pragma unroll
        for (int n = 0; n < MR / 4; ++n) {
          const int r = 4 * n + srow;
          const u32x4_t v = *reinterpret_cast<lds_cu32x4*>(W + r * 256 + ((sch ^ swz_c(r)) * 16));
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(dst + (int64_t)r * g.ldc + sch * 8));
        }
      }
    }
    stores += TJ * (4 / QR) * (MR / 4);
  }
  return stores;
}

// NKC: K units known at compile time (16: K = 512, the tile_size 512 case;
// 0: K from the arguments). NW: waves per workgroup (4 or 8).
template <int MODE, int NKC, int NW, bool SC>
__global__ __launch_bounds__(64 * NW, 1) void ns_st_kernel(StArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kSlots<MODE> * SLOT];
  const int nbi = g.M / BT, nbj = g.N / BT;
  const int per_tile = (MODE == kApply) ? nbi * nbj : nbi * (nbi + 1) / 2;
  const int64_t total = g.ntiles * per_tile;
  const int wper = (int)(gridDim.x >> 3);
  const int64_t per_xcd = (total + 7) >> 3;
  const int64_t ibeg = (int64_t)(blockIdx.x & 7) * per_xcd;
  const int64_t iend = (ibeg + per_xcd < total) ? ibeg + per_xcd : total;
  auto pos = [&](int64_t item) {
    ItemPos q;
    q.tile = item / per_tile;
    const int p = (int)(item - q.tile * per_tile);
    if constexpr (MODE == kApply) {
      q.bi = p / nbj;
      q.bj = p - q.bi * nbj;
      q.diag = false;
    } else {
      int bi = 0;
      while ((bi + 1) * (bi + 2) / 2 <= p) ++bi;
      q.bi = bi;
      q.bj = p - bi * (bi + 1) / 2;
      q.diag = q.bi == q.bj;
    }
    return q;
  };
  int64_t item = ibeg + (blockIdx.x >> 3);
  if (item >= iend) return;
  ItemPos cur = pos(item);
  int pre_st = 0;
  for (;;) {
    const int64_t next = item + wper;
    const bool more = next < iend;
    const ItemPos nxt = pos(more ? next : item);
    const int st = cur.diag ? st_item<MODE, true, NKC, NW, SC>(g, (lds_u8*)lds, cur, pre_st, more, nxt)
                            : st_item<MODE, false, NKC, NW, SC>(g, (lds_u8*)lds, cur, pre_st, more, nxt);
    if (!more) break;
    pre_st = st;
    item = next;
    cur = nxt;
  }
}

// CUs of the current device, queried per launch (a host-side attribute
// lookup; nothing is cached in the library).
int num_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

template <int MODE, bool SC = false>
void launch(const StArgs& a, int64_t items, hipStream_t s) {
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t wgs_per_xcd = std::max<int64_t>(1, std::min<int64_t>(num_cus() / 8, per_xcd));
  const dim3 grid((unsigned)(8 * wgs_per_xcd));
  // 8 waves (two per SIMD): 4.5 % faster than 4 at K = 512 and about 10 %
  // at K = 256 and 1024 on MI355X, so only that layout is launched.
  constexpr int kNW = 8;
  if (a.K == 16 * BK)
    hipLaunchKernelGGL((ns_st_kernel<MODE, 16, kNW, SC>), grid, dim3(64 * kNW), 0, s, a);
  else
    hipLaunchKernelGGL((ns_st_kernel<MODE, 0, kNW, SC>), grid, dim3(64 * kNW), 0, s, a);
}

}  // namespace

bool ns5_stream_supported(int mp, int np) { return mp % BT == 0 && np % BT == 0; }

void ns_stream_product(int mode, const uint16_t* P, int64_t p_bs, int ldp, const uint16_t* Q, int64_t q_bs,
                       int ldq, const uint16_t* R, int64_t r_bs, int ldr, uint16_t* C, int64_t c_bs, int ldc,
                       int M, int N, int K, int64_t ntiles, float alpha, float beta, bool round_once,
                       hipStream_t s) {
  const StArgs g{P, p_bs, ldp, Q, q_bs, ldq, R, r_bs, ldr, C, c_bs, ldc, M, N, K, ntiles, alpha, beta,
                 round_once ? 1 : 0, nullptr};
  const int nb = M / BT;
  if (mode == kApply)
    launch<kApply>(g, ntiles * nb * (N / BT), s);
  else if (mode == kGramB)
    launch<kGramB>(g, ntiles * (nb * (nb + 1) / 2), s);
  else
    launch<kGramA>(g, ntiles * (nb * (nb + 1) / 2), s);
}

// One sub-batch of `cnt` tiles, `steps` >= 1 iterations, ping-ponging X
// between x and y; the first iteration's kernels scale the raw x on load
// (X0 is never written); A and B live in the workspace.
int ns5_stream_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                   float a, float b, float c, bool round_once, bool fused_ba, uint16_t* wsA, uint16_t* wsB,
                   hipStream_t s, const BaUntile* untile) {
  if (fused_ba && cnt > kBaMaxTiles) return HIMUON_EINVAL;
  if (untile && (!fused_ba || steps < 2)) return HIMUON_EINVAL;
  const int64_t sq = (int64_t)mp * mp, rect = (int64_t)mp * np;
  const int nb = mp / BT;
  const int64_t gram_items = cnt * (nb * (nb + 1) / 2);
  const int64_t apply_items = cnt * nb * (np / BT);
  uint16_t* cur = x;
  uint16_t* nxt = y;
  for (int it = 0; it < steps; ++it) {
    const float* xinv = it == 0 ? inv : nullptr;
    const StArgs ga{cur, rect, np, cur, rect, np, nullptr, 0, 0, wsA, sq, mp, mp, mp, np, cnt, 1.0f, 0.0f, 0, xinv};
    if (xinv)
      launch<kGramA, true>(ga, gram_items, s);
    else
      launch<kGramA>(ga, gram_items, s);
    if (fused_ba) {  // B stays on chip: ns5_ba.hip
      // the untile fused into the last iteration; its per-tile records go to
      // wsB, which the fused path does not use otherwise (cnt mp^2 bf16)
      BaUntile u{};
      if (untile && it + 1 == steps) {
        u = *untile;
        u.rec = reinterpret_cast<int32_t*>(wsB);
      }
      if (!ns5_ba_run(wsA, cur, nxt, xinv, cnt, a, b, c, round_once, s, u.params ? &u : nullptr))
        return HIMUON_EINVAL;
      std::swap(cur, nxt);
      continue;
    }
    const StArgs gb{wsA, sq, mp, wsA, sq, mp, wsA, sq, mp, wsB, sq, mp, mp, mp, mp, cnt, c, b, 0, nullptr};
    launch<kGramB>(gb, gram_items, s);
    const StArgs ap{wsB, sq, mp, cur, rect, np, cur, rect, np, nxt, rect, np, mp, np, mp, cnt, 1.0f, a,
                    round_once ? 1 : 0, xinv};
    if (xinv)
      launch<kApply, true>(ap, apply_items, s);
    else
      launch<kApply>(ap, apply_items, s);
    std::swap(cur, nxt);
  }
  return 0;
}
