// NS5 stages for 512x512 NS tiles (tile_size 512): one persistent kernel per
// stage whose operand stream never drains between output blocks.
//
//   GramA : C = A = bf16(X X^T)            P = Q = X               lower blocks + mirror
//   GramB : C = B = bf16(c A A^T + b A)    P = Q = A               lower blocks + mirror
//   Apply : C = X' = bf16(bf16(B X) + a X) P = B, Q = X read as [k][j]
// (ns5_smem.py:89-101, XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88).
// Every operand is 512x512 with row pitch 512; K = 512 is 16 units of 32.
//
// One 256-thread workgroup per CU (4 waves in 2x2, each a 128x128 sub-block of
// 4x4 v_mfma_f32_32x32x16_bf16 tiles; operands swapped so lane l holds
// C[row l%32][4 consecutive columns]) walks a contiguous range of 256x256
// output blocks of its XCD. LDS (160 KiB) is a 4-slot ring of 32 KiB operand
// units plus one 32 KiB staging slot.
//
// * Operand stream: units go straight from global memory into the ring
//   (global_load_lds_dwordx4), 3 units ahead of the MFMAs, and the stream runs
//   on into the next block's first units, so a block starts with its operands
//   already in LDS.
// * Epilogue operand: the R = A (GramB) or X (Apply) block passes through the
//   ring as part of P (GramB) or Q (Apply). The K order of a block is rotated
//   so that those 8 units come last, and each wave copies its 128x128 part of
//   R from them into registers.
// * Stores: the finished block is converted to bf16 and kept in registers;
//   during the first 8 units of the next block each wave stages one 32-row
//   stripe per unit in its quarter of the staging slot and writes it with
//   16-byte row-contiguous stores (4 rows x 256 bytes per instruction), the
//   mirrored block of an off-diagonal Gram block in 4 more stripes (4x4
//   transposes across lane quads). The stores drain behind the MFMAs.
// * Waits: vmcnt retires loads and stores in issue order, so waiting for unit u
//   with vmcnt(#loads of the next 2 units + #stores issued after unit u) is
//   exact.
#include "ns5_kernels.h"

namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) const u32x4_t lds_cu32x4;
typedef __attribute__((address_space(3))) const u32x2_t lds_cu32x2;
typedef __attribute__((address_space(3))) u32x2_t lds_u32x2;

constexpr int NT = 256;
constexpr int T = 512;                 // tile edge = K = row pitch of every operand
constexpr int BT = 256;                // output block edge
constexpr int BK = 32;                 // K per stream unit
constexpr int NK = T / BK;             // 16 units per block
constexpr int SLOT = 32768;            // bytes per ring slot
constexpr int NRING = 4;               // ring slots
constexpr int DIST = NRING - 1;        // units in flight ahead of the MFMAs
constexpr int HALF = SLOT / 2;         // Q panel offset within a slot
constexpr int STAGE = NRING * SLOT;    // staging slot offset
constexpr int LDS_BYTES = STAGE + SLOT;
constexpr int NPARK = 8;               // units that carry the previous block's stores

enum { kGramA = 0, kGramB = 1, kApply = 2 };

struct T5Args {
  const uint16_t* P;  // rows i, k-contiguous (X, A or B)
  const uint16_t* Q;  // Gram: rows j, k-contiguous; Apply: X as [k][j]
  uint16_t* C;        // output
  int64_t ntiles;
  float alpha, beta;  // GramB: c, b; Apply: beta = a
};

HM_DEV f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

HM_DEV uint32_t pk_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t r;
  r[0] = (__bf16)lo;
  r[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

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
// vmcnt(n) for a wave-uniform n in {0, 4, ..., 48}; anything else waits for 0.
HM_DEV void wait_vm_n(int n) {
  switch (n) {
    case 4: wait_vm<4>(); break;
    case 8: wait_vm<8>(); break;
    case 12: wait_vm<12>(); break;
    case 16: wait_vm<16>(); break;
    case 20: wait_vm<20>(); break;
    case 24: wait_vm<24>(); break;
    case 28: wait_vm<28>(); break;
    case 32: wait_vm<32>(); break;
    case 36: wait_vm<36>(); break;
    case 40: wait_vm<40>(); break;
    case 44: wait_vm<44>(); break;
    case 48: wait_vm<48>(); break;
    default: wait_vm<0>(); break;
  }
}

// Workgroup barrier for LDS reuse (this wave's LDS operations complete; global
// memory operations stay in flight and are waited for with vmcnt).
HM_DEV void lds_barrier() {
  wait_lgkm<0>();
  asm volatile("s_barrier" ::: "memory");
}

// Direct-to-LDS 16-byte load: lane l's 16 bytes from base + voff (base
// wave-uniform, in SGPRs; voff a 32-bit lane byte offset) land at
// lds_wave + 16 l. Issued as inline assembly so that the compiler's waitcnt
// model, which treats the builtin as a flat access to global memory and LDS,
// does not force full waits before unrelated LDS reads.
HM_DEV void dma16(const uint16_t* base, uint32_t voff, uint32_t lds_wave) {
  // readfirstlane returns int: widen through uint32_t (a sign-extended low
  // word would set the upper 32 address bits).
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint64_t ub = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)) << 32) |
                      (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(ub), "s"(__builtin_amdgcn_readfirstlane(lds_wave))
      : "memory", "m0");
}

// ds_read_b64_tr_b16 (inline assembly, see dma16); valid after an lgkmcnt wait.
HM_DEV u32x2_t ds_read_tr16(uint32_t addr) {
  u32x2_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

HM_DEV uint32_t quad_swap2(uint32_t v) { return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false); }
HM_DEV uint32_t quad_swap1(uint32_t v) { return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false); }

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

// Chunk swizzles (16-byte chunk index XOR a function of the row).
// P/Q row panels (64-byte rows): fragment reads of 8/16 consecutive rows
// of one chunk hit distinct bank groups.
HM_DEV int swz_p(int r) { return (((r >> 1) ^ (r >> 3)) & 1) | (((r >> 2) & 1) << 1); }
// X panel of Apply (512-byte rows): a function of r & 3 spreads the
// transposing reads (4 rows x 32 bytes per 16 lanes); the r >> 2 part is
// constant within each such read and makes 32 consecutive rows of one chunk
// (the R copy) land on 32 distinct positions.
HM_DEV int swz_x(int r) {
  return (10 * (r & 1) + 4 * ((r >> 1) & 1)) ^ ((r >> 2) & 1) ^ (((r >> 3) & 1) << 4) ^
         (((r >> 4) & 1) << 1);
}
// Output staging (256-byte rows).
HM_DEV int swz_c(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// One output block of a stage.
struct Item {
  int64_t tile;
  int bi, bj;
  bool diag;  // Gram diagonal block: Q = P, no mirror
  bool valid;
};

template <int MODE>
HM_DEV Item decode(int64_t item, int64_t iend) {
  Item it;
  it.valid = item < iend;
  constexpr int per_tile = (MODE == kApply) ? 4 : 3;
  const int64_t t = it.valid ? item / per_tile : 0;
  const int p = it.valid ? (int)(item - t * per_tile) : 0;
  it.tile = t;
  if constexpr (MODE == kApply) {
    it.bi = p >> 1;
    it.bj = p & 1;
    it.diag = false;
  } else {  // (0,0), (1,0), (1,1)
    it.bi = p > 0;
    it.bj = p > 1;
    it.diag = p != 1;
  }
  return it;
}

template <int MODE>
__global__ __launch_bounds__(NT, 1) void ns_t512_kernel(T5Args g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[LDS_BYTES];
  constexpr bool kTr = MODE == kApply;
  constexpr bool kR = MODE != kGramA;  // epilogue operand copied from the stream
  constexpr int per_tile = kTr ? 4 : 3;
  const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds_raw;

  // Per-lane constants. The thread index is made opaque once per stream unit
  // (lane_setup) so that the many per-lane LDS/global offsets derived from it
  // (XOR swizzles do not fold into instruction offsets) are recomputed where
  // they are used instead of being kept live across the block, where they
  // would not fit in registers next to the fragments and parked outputs.
  int tid = threadIdx.x;
  int lane = tid & 63, wave = tid >> 6;
  int wm = wave >> 1, wn = wave & 1;
  int l32 = lane & 31, hi = lane >> 5;

  const int64_t total = g.ntiles * per_tile;
  const int wper = (int)(gridDim.x >> 3);
  const int64_t per_xcd = (total + 7) >> 3;
  const int64_t ibeg = (int64_t)(blockIdx.x & 7) * per_xcd;
  const int64_t iend = (ibeg + per_xcd < total) ? ibeg + per_xcd : total;
  int64_t item = ibeg + (blockIdx.x >> 3);
  if (item >= iend) return;

  int prl, pch, xr, sp, r16, te, tr_row, tr_chunk, tr_sub, srow, sch;
  uint32_t voff_p, prow, qrow, wdst, stage;
  uint32_t voff_x[4];
  auto lane_setup = [&]() {
    asm volatile("" : "+v"(tid));
    lane = tid & 63;
    wave = tid >> 6;
    wm = wave >> 1;
    wn = wave & 1;
    l32 = lane & 31;
    hi = lane >> 5;
    prl = lane >> 2;                         // row-panel loader: row within 16
    pch = (lane & 3) ^ swz_p(prl);           //   and fetched chunk
    voff_p = ((16 * wave + prl) * T + pch * 8) * 2;
    xr = 2 * wave + hi;                      // X-panel loader: row within 8
#pragma unroll
    for (int i = 0; i < 4; ++i) voff_x[i] = (xr * T + ((l32 ^ swz_x(8 * i + xr)) * 8)) * 2;
    sp = swz_p(l32 & 15);
    prow = (wm * 128 + l32) * 64;
    qrow = (wn * 128 + l32) * 64;
    r16 = lane & 15;
    te = r16 >> 2;
    tr_row = 8 * hi + te;
    tr_chunk = wn * 16 + 2 * ((lane >> 4) & 1) + ((r16 & 3) >> 1);
    tr_sub = (r16 & 1) * 8;
    wdst = lds + wave * 1024;
    stage = lds + STAGE + wave * 8192;       // this wave's 8 KiB staging stripe
    srow = lane >> 4;
    sch = lane & 15;
  };
  lane_setup();

  // K rotation: the 8 units holding the epilogue operand come last.
  auto rot_of = [&](const Item& it) -> int {
    if constexpr (MODE == kApply) return it.bi ? 0 : 8;
    else if constexpr (MODE == kGramB) return it.bj ? 0 : 8;
    else return 0;
  };

  // Issue stream unit u (0..15) of item `it` into ring slot `slot`.
  auto issue = [&](const Item& it, int u, int slot) {
    const int kidx = (u + rot_of(it)) & (NK - 1);
    const uint32_t d = wdst + slot * SLOT;
    const uint16_t* pb = g.P + it.tile * (int64_t)(T * T) + (int64_t)(it.bi * BT) * T + kidx * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(pb + i * 64 * T, voff_p, d + i * 4096);
    if constexpr (kTr) {
      const uint16_t* qb = g.Q + it.tile * (int64_t)(T * T) + (int64_t)(kidx * BK) * T + it.bj * BT;
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16(qb + i * 8 * T, voff_x[i], d + HALF + i * 4096);
    } else {
      if (!it.diag) {
        const uint16_t* qb = g.Q + it.tile * (int64_t)(T * T) + (int64_t)(it.bj * BT) * T + kidx * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(qb + i * 64 * T, voff_p, d + HALF + i * 4096);
      }
    }
  };

  // Fragments of the unit in `slot`, sub-step ks.
  auto frags = [&](int slot, int ks, bool diag, u32x4_t(&fa)[4], u32x4_t(&fb)[4]) {
    const uint32_t s = lds + slot * SLOT;
    const uint32_t pos = ((2 * ks + hi) ^ sp) * 16;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      fb[t] = *reinterpret_cast<lds_cu32x4*>((uintptr_t)(s + prow + t * 2048 + pos));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if constexpr (kTr) {
        const int row = 16 * ks + tr_row;  // row & 31; rows row and row + 4
        const uint32_t off = s + HALF + row * 512 + (((tr_chunk + 4 * t) ^ swz_x(row)) * 16) + tr_sub;
        const uint32_t off2 = s + HALF + (row + 4) * 512 + (((tr_chunk + 4 * t) ^ swz_x(row + 4)) * 16) + tr_sub;
        const u32x2_t l2 = ds_read_tr16(off), u2 = ds_read_tr16(off2);
        fa[t] = u32x4_t{l2[0], l2[1], u2[0], u2[1]};
      } else {
        const uint32_t qs = diag ? s : s + HALF;
        fa[t] = *reinterpret_cast<lds_cu32x4*>((uintptr_t)(qs + qrow + t * 2048 + pos));
      }
    }
  };

  f32x16_t acc[4][4];
  auto mma = [&](const u32x4_t(&fa)[4], const u32x4_t(&fb)[4]) {
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
  };

  // Epilogue operand copy of unit 8 + p (p = 0..7) in `slot`: GramB takes
  // A[i][j] from the P panel (columns = this unit's k), Apply takes X[i][j]
  // from the X panel (rows = this unit's k). Units p < 4 hold the part of the
  // waves with wn (GramB) / wm (Apply) = 0, units p >= 4 that of the others;
  // every wave copies the first and the owners overwrite from the second, so
  // that each register is written unconditionally within the block and dies
  // in its epilogue.
  u32x2_t rv[4][4][4];
  auto capture = [&](int slot, int p) {
    const int idx = p & 3;
    const uint32_t s = lds + slot * SLOT;
    const bool mine = ((MODE == kGramB) ? wn : wm) == (p >> 2);
    if constexpr (MODE == kGramB) {
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (p < 4 || mine)
            rv[ti][idx][q] =
                *reinterpret_cast<lds_cu32x2*>((uintptr_t)(s + prow + ti * 2048 + ((q ^ sp) * 16) + hi * 8));
        }
    } else if constexpr (MODE == kApply) {
      const int sx = swz_x(l32);
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int ch = wn * 16 + 4 * tj + q;
          if (p < 4 || mine)
            rv[idx][tj][q] =
                *reinterpret_cast<lds_cu32x2*>((uintptr_t)(s + HALF + l32 * 512 + ((ch ^ sx) * 16) + hi * 8));
        }
    }
  };

  // Parked output of the previous block (bf16, C[i][j..j+3] per (ti, tj, q))
  // and its store passes: the 32-row stripes of C and, for off-diagonal Gram
  // blocks, those of the mirrored block.
  u32x2_t pc[4][4][4];
  Item prev{0, 0, 0, true, false};
  int np_prev = 0;
  // store_pass(p, mirror_pass): C stripe p, or mirror stripe p. Called with
  // arguments that are constants after unrolling (a runtime index into pc
  // would put pc in scratch memory).
  auto store_pass = [&](int p, bool mirror_pass) {
    uint16_t* base;
    if (!mirror_pass) {
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = l32, ch = 4 * tj + q;
          *reinterpret_cast<lds_u32x2*>((uintptr_t)(stage + r * 256 + ((ch ^ swz_c(r)) * 16) + hi * 8)) =
              pc[p][tj][q];
        }
      base = g.C + prev.tile * (int64_t)(T * T) + (int64_t)(prev.bi * BT + wm * 128 + 32 * p) * T + prev.bj * BT +
             wn * 128;
    } else {
      const int tj = p, k = lane & 3, a = l32 >> 2;
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x2_t tv = quad_transpose(pc[ti][tj][q], k);
          const int r = 8 * q + 4 * hi + k, ch = 4 * ti + (a >> 1);
          *reinterpret_cast<lds_u32x2*>((uintptr_t)(stage + r * 256 + ((ch ^ swz_c(r)) * 16) + (a & 1) * 8)) = tv;
        }
      base = g.C + prev.tile * (int64_t)(T * T) + (int64_t)(prev.bj * BT + wn * 128 + 32 * tj) * T + prev.bi * BT +
             wm * 128;
    }
    wait_lgkm<0>();
    const uint32_t soff = (srow * T + sch * 8) * 2;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int r = 4 * n + srow;
      const u32x4_t v = *reinterpret_cast<lds_cu32x4*>((uintptr_t)(stage + r * 256 + ((sch ^ swz_c(r)) * 16)));
      *reinterpret_cast<u32x4_t*>(reinterpret_cast<char*>(base + 4 * n * T) + soff) = v;
      if (n & 1) __builtin_amdgcn_sched_barrier(0);  // at most 2 stripe rows in registers
    }
  };

  // ---- stream --------------------------------------------------------------
  Item cur = decode<MODE>(item, iend);
  Item nxt = decode<MODE>(item + wper, iend);
#pragma unroll
  for (int u = 0; u < DIST; ++u) issue(cur, u, u);

  while (true) {
    lane_setup();
    const int lk = cur.diag ? 4 : 8;                     // loads per wave of a unit of this block
    const int ln = nxt.valid ? (nxt.diag ? 4 : 8) : 0;   // ... of the next block
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

    u32x4_t fa0[4], fb0[4], fa1[4], fb1[4];
#pragma unroll
    for (int u = 0; u < NK; ++u) {
      lane_setup();  // recompute the per-lane offsets for this unit (see lane_setup)
      // Unit u has landed: the loads of units u + 1, u + 2 and the stores
      // of the passes issued after it (iterations u - 3 .. u - 1) are younger.
      int n = ((u + 1 < NK) ? lk : ln) + ((u + 2 < NK) ? lk : ln);
#pragma unroll
      for (int x = u - 3; x < u; ++x)
        if (x >= 0 && x < np_prev) n += 8;
      wait_vm_n(n);
      lds_barrier();  // unit u is visible; slot (u - 1) % NRING is free
      // unit u + 3 (of this block or the next) into the freed slot
      if (u + DIST < NK)
        issue(cur, u + DIST, (u + DIST) % NRING);
      else if (nxt.valid)
        issue(nxt, u + DIST - NK, (u + DIST) % NRING);
      frags(u % NRING, 0, cur.diag, fa0, fb0);
      if (u > 0) {  // second half of unit u - 1, covering the reads above
        __builtin_amdgcn_sched_barrier(0);
        mma(fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
      }
      // pass u of the previous block: C stripes 0..3 (4 passes) or, for an
      // off-diagonal Gram block, C and mirror stripes interleaved (8 passes)
      if (u < NPARK) {
        if (np_prev == 8)
          store_pass(u >> 1, u & 1);
        else if (u < 4 && np_prev == 4)
          store_pass(u, false);
      }
      if (kR && u >= NK - 8) capture(u % NRING, u - (NK - 8));
      wait_lgkm<0>();
      frags(u % NRING, 1, cur.diag, fa1, fb1);
      __builtin_amdgcn_sched_barrier(0);
      mma(fa0, fb0);
      __builtin_amdgcn_sched_barrier(0);
      wait_lgkm<0>();  // this wave is done with slot u % NRING
    }
    mma(fa1, fb1);

    // Epilogue: park the block as bf16.
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x16_t& v = acc[tj][ti];
          if constexpr (MODE == kGramA) {
            pc[ti][tj][q] = u32x2_t{pk_bf16(v[4 * q], v[4 * q + 1]), pk_bf16(v[4 * q + 2], v[4 * q + 3])};
          } else {
            const u32x2_t r = rv[ti][tj][q];
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float x = bf16_to_f32(half16(r[e >> 1], e & 1));
              if constexpr (MODE == kApply)
                y[e] = fmaf(g.beta, x, bf16_to_f32(pk_bf16(v[4 * q + e], 0.f) & 0xffffu));  // bf16(B X) + a X
              else
                y[e] = fmaf(g.beta, x, g.alpha * v[4 * q + e]);  // c (A A^T) + b A
            }
            pc[ti][tj][q] = u32x2_t{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
          }
        }
    prev = cur;
    np_prev = (MODE == kApply || cur.diag) ? 4 : 8;
    if (!nxt.valid) break;
    item += wper;
    cur = nxt;
    nxt = decode<MODE>(item + wper, iend);
  }
  // The last block's stores.
  if (np_prev == 8) {
#pragma unroll
    for (int p = 0; p < 8; ++p) store_pass(p >> 1, p & 1);
  } else if (np_prev == 4) {
#pragma unroll
    for (int p = 0; p < 4; ++p) store_pass(p, false);
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
void launch(const T5Args& a, int64_t items, hipStream_t s) {
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t wgs_per_xcd = std::max<int64_t>(1, std::min<int64_t>(num_cus() / 8, per_xcd));
  hipLaunchKernelGGL((ns_t512_kernel<MODE>), dim3((unsigned)(8 * wgs_per_xcd)), dim3(NT), 0, s, a);
}

// X0 = bf16(x * inv) in place, 8 elements per thread.
__global__ __launch_bounds__(NT) void ns_t512_scale_kernel(uint16_t* __restrict__ x, const float* __restrict__ inv,
                                                           int64_t ntiles) {
  const int64_t nvec = ntiles * (T * T / 8);
  for (int64_t v = (int64_t)blockIdx.x * NT + threadIdx.x; v < nvec; v += (int64_t)gridDim.x * NT) {
    u32x4_t* p = reinterpret_cast<u32x4_t*>(x) + v;
    *p = scale8(*p, inv[v / (T * T / 8)]);
  }
}

}  // namespace

bool ns5_t512_supported(int mp, int np) { return mp == T && np == T; }

// One sub-batch of `cnt` 512x512 tiles, `steps` >= 1 iterations, X
// ping-ponging between x and y (x is scaled in place first); A and B live in
// the workspace.
void ns5_t512_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int steps, float a, float b, float c,
                  uint16_t* wsA, uint16_t* wsB, hipStream_t s) {
  const int64_t nvec = cnt * (T * T / 8);
  hipLaunchKernelGGL(ns_t512_scale_kernel, dim3((unsigned)std::min<int64_t>((nvec + NT - 1) / NT, 65536)), dim3(NT),
                     0, s, x, inv, cnt);
  uint16_t* cur = x;
  uint16_t* nxt = y;
  for (int it = 0; it < steps; ++it) {
    launch<kGramA>(T5Args{cur, cur, wsA, cnt, 1.0f, 0.0f}, cnt * 3, s);
    launch<kGramB>(T5Args{wsA, wsA, wsB, cnt, c, b}, cnt * 3, s);
    launch<kApply>(T5Args{wsB, cur, nxt, cnt, 1.0f, a}, cnt * 4, s);
    std::swap(cur, nxt);
  }
}
