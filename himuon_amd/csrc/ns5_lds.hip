// Fused Newton-Schulz for NS tiles with mp == 128 and np in {128, 256, 512}:
// one workgroup keeps a tile's X (128 x np) and its A / B (128 x 128) in LDS
// through all iterations, so HBM sees one read and one write of the tile.
// This is the LDS-resident counterpart of the reference's one-kernel NS5 for
// small tiles (triton_kernels/ns5_smem.py:46-104, dispatched for M*N <= 16384
// by himuon.py:263-284); the per-iteration rounding points are those of the
// three-kernel path (XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88):
//
//   X0 = bf16(x * inv)
//   A  = bf16(X X^T)                    lower 32x32 tiles only
//   B  = bf16(c (A A^T) + b A)          lower 32x32 tiles only
//   X' = bf16(bf16(B X) + a X)
//
// np = 128: 256 threads = 4 waves, three workgroups per CU; np = 256, 512:
// 512 threads = 8 waves, two per SIMD (one workgroup fits a CU). Gram
// products: the 10 lower 32x32 tiles (ti >= tj of the 4x4 grid of
// v_mfma_f32_32x32x16_bf16 tiles) are split 3, 3, 2, 2 over the four waves
// (GramPart), or over eight waves with the same 3, 3, 2, 2 per SIMD
// (GramPart8), so every SIMD takes part. A and B are symmetric
// and only those 10 tiles are stored (20 KiB): a row fragment of an upper
// tile (i, k), k > i, is read from the stored tile (k, i) with the
// contraction along its rows. A diagonal tile is computed whole and is
// exactly symmetric (element (i, j) and (j, i) sum the same products in the
// same order), and an off-diagonal tile read transposed holds the values its
// mirror would, so every operand is the full matrix's, bit for bit. Apply:
// wave w of NW owns columns w np/NW .. + np/NW - 1 of all 128 rows (in passes
// of at most 64 columns) and writes X' over its own columns of X as each pass
// ends. Every output element sums its k terms in one accumulator in the same
// order whatever the wave count, so both forms give the same bits.
// Products accumulate in registers; B replaces A after a workgroup barrier.
// X is read as the MFMA B operand with the contraction along its rows through
// ds_read_b64_tr_b16.
// The next tile's X is loaded into registers while the current tile iterates.
// The k loops are unrolled fully, so the compiler issues later fragment reads
// ahead of the MFMAs that need them (7 % faster than 2- and 4-fold unrolling).
//
// X rows hold 16-byte chunks; chunk ch of row r sits at position
// ch ^ s(r), s(r) = 4 (r % 4) + (r / 4) % 4: 16 consecutive rows of one chunk
// (fragment reads) and 4 consecutive rows of 4 consecutive chunks
// (transposing reads) both cover all 16 bank groups. A stored 32x32 tile has
// 64-byte rows, chunk ch of row r at ch ^ ((r / 4) % 4): 16 consecutive rows
// of one chunk and 4 consecutive rows of 2 chunks hit distinct bank groups.
// np = 128: 52 KiB per workgroup, three workgroups per CU; np = 256: 84 KiB,
// np = 512: 148 KiB, one per CU (eight waves).
#include "elem_ops.h"
#include "ns5_kernels.h"

namespace {

constexpr int NT = 256;
constexpr int M = 128;  // NS rows (mp)

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) u32x4_t lds_u32x4;

HM_DEV uint32_t lds_pos(int r, int ch, int chunks) {
  const int sw = ((r & 3) << 2) | ((r >> 2) & 3);
  return (uint32_t)(r * chunks + (ch ^ sw)) * 16u;
}

// Stored lower 32x32 tile (ti >= tj) of a symmetric 128 x 128 matrix:
// byte offset of 16-byte chunk ch (columns 8 ch ..) of its row r.
constexpr int TRI_TILE = 32 * 32 * 2;
constexpr int TRI_BYTES = 10 * TRI_TILE;
HM_DEV uint32_t tri_pos(int ti, int tj, int r, int ch) {
  return (uint32_t)((ti * (ti + 1) / 2 + tj) * TRI_TILE + r * 64 + ((ch ^ ((r >> 2) & 3)) << 4));
}

// Transposing read: 4 bf16 of the 8-byte row segment at `off`, redistributed
// across each group of 16 lanes (lane 4a + b receives element b of the
// segments addressed by lanes a, a + 4, a + 8, a + 12).
HM_DEV u32x2_t read_tr(const lds_u8* base, uint32_t off) {
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base + off));
  return __builtin_bit_cast(u32x2_t, r);
}

// The lane index, opaque to the optimiser: addresses derived from it are
// formed inside each phase instead of being hoisted out of the iteration loop
// for all four per-wave variants at once (which would not fit the registers).
HM_DEV int opaque_lane(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Row fragment of a symmetric matrix S stored as its lower tiles: lane (l32,
// hi) receives S[32 R + l32][16 ks + 8 hi .. + 7] (the MFMA operand of row
// tile R, k-step ks). Column tile k = ks / 2 > R is read from the stored tile
// (k, R) as the transposing reads of the X operand do.
template <int R, int KS>
HM_DEV u32x4_t tri_frag(const lds_u8* S, int l32, int hi, int tr_krow, int tr_col) {
  constexpr int TK = KS >> 1;
  if constexpr (TK <= R) {
    return *reinterpret_cast<lds_cu32x4*>(S + tri_pos(R, TK, l32, 2 * (KS & 1) + hi));
  } else {
    const int kr = 16 * (KS & 1) + tr_krow;
    const u32x2_t l2 = read_tr(S, tri_pos(TK, R, kr, tr_col >> 3) + (tr_col & 7) * 2);
    const u32x2_t u2 = read_tr(S, tri_pos(TK, R, kr + 4, tr_col >> 3) + (tr_col & 7) * 2);
    return u32x4_t{l2[0], l2[1], u2[0], u2[1]};
  }
}

// Transposing-read lane roles (the X operand of Apply, the upper fragments of
// A and B): lane (a', b') of each 16-lane group addresses k-row 8 hi + a' (+ 4
// for the second read) and columns 16 ((lane >> 4) & 1) + 4 b' .. + 3 of a
// 32-column tile.
HM_DEV int tr_krow_of(int lane) { return 8 * (lane >> 5) + ((lane & 15) >> 2); }
HM_DEV int tr_col_of(int lane) { return 16 * ((lane >> 4) & 1) + 4 * (lane & 3); }

// Wave W's share of a Gram product's lower 32x32 tiles: it loads the row tiles
// ROW[0 .. NR-1] of the operand and computes tiles k < NTL, tile k being
// (row tile ROW[I[k]], column tile ROW[J[k]]).
template <int W> struct GramPart;
template <> struct GramPart<0> {  // (0,0) (1,0) (1,1)
  static constexpr int NR = 2, NTL = 3, ROW[3] = {0, 1, 0}, I[3] = {0, 1, 1}, J[3] = {0, 0, 1};
};
template <> struct GramPart<1> {  // (2,0) (2,1) (2,2)
  static constexpr int NR = 3, NTL = 3, ROW[3] = {0, 1, 2}, I[3] = {2, 2, 2}, J[3] = {0, 1, 2};
};
template <> struct GramPart<2> {  // (3,0) (3,1)
  static constexpr int NR = 3, NTL = 2, ROW[3] = {0, 1, 3}, I[3] = {2, 2, 0}, J[3] = {0, 1, 0};
};
template <> struct GramPart<3> {  // (3,2) (3,3)
  static constexpr int NR = 2, NTL = 2, ROW[3] = {2, 3, 0}, I[3] = {1, 1, 0}, J[3] = {0, 1, 0};
};
// The same 10 tiles over eight waves (two per SIMD; wave w shares SIMD w % 4
// with wave w + 4): the diagonal tiles in pairs, the off-diagonal ones alone,
// so a SIMD still computes 3, 3, 2, 2 tiles. Each tile sums its k terms in
// one accumulator in the same order as the four-wave split.
template <int W> struct GramPart8;
template <> struct GramPart8<0> {  // (0,0) (1,1)
  static constexpr int NR = 2, NTL = 2, ROW[3] = {0, 1, 0}, I[3] = {0, 1, 0}, J[3] = {0, 1, 0};
};
template <> struct GramPart8<1> {  // (2,2) (3,3)
  static constexpr int NR = 2, NTL = 2, ROW[3] = {2, 3, 0}, I[3] = {0, 1, 0}, J[3] = {0, 1, 0};
};
template <int TI, int TJ> struct GramPartOne {  // (TI, TJ), TI > TJ
  static constexpr int NR = 2, NTL = 1, ROW[3] = {TI, TJ, 0}, I[3] = {0, 0, 0}, J[3] = {1, 0, 0};
};
template <> struct GramPart8<2> : GramPartOne<1, 0> {};
template <> struct GramPart8<3> : GramPartOne<2, 0> {};
template <> struct GramPart8<4> : GramPartOne<2, 1> {};
template <> struct GramPart8<5> : GramPartOne<3, 0> {};
template <> struct GramPart8<6> : GramPartOne<3, 1> {};
template <> struct GramPart8<7> : GramPartOne<3, 2> {};

// Calls f(part) with wave `wave`'s share of a Gram product (NW = 4 or 8).
template <int NW, class F>
HM_DEV void with_part(int wave, F&& f) {
  if constexpr (NW == 4) {
    switch (wave) {
      case 0: f(GramPart<0>{}); break;
      case 1: f(GramPart<1>{}); break;
      case 2: f(GramPart<2>{}); break;
      default: f(GramPart<3>{}); break;
    }
  } else {
    switch (wave) {
      case 0: f(GramPart8<0>{}); break;
      case 1: f(GramPart8<1>{}); break;
      case 2: f(GramPart8<2>{}); break;
      case 3: f(GramPart8<3>{}); break;
      case 4: f(GramPart8<4>{}); break;
      case 5: f(GramPart8<5>{}); break;
      case 6: f(GramPart8<6>{}); break;
      default: f(GramPart8<7>{}); break;
    }
  }
}

// Fragments of row tile R at k-step KS: from X (SCH chunks per row) or, TRI,
// from a symmetric matrix stored as its lower tiles.
template <bool TRI, int SCH, int R, int KS>
HM_DEV u32x4_t row_frag(const lds_u8* S, int l32, int hi, int tr_krow, int tr_col) {
  if constexpr (TRI)
    return tri_frag<R, KS>(S, l32, hi, tr_krow, tr_col);
  else
    return *reinterpret_cast<lds_cu32x4*>(S + lds_pos(32 * R + l32, 2 * KS + hi, SCH));
}

template <class P, bool TRI, int SCH, int KS>
HM_DEV void gram_step(const lds_u8* S, int l32, int hi, int tr_krow, int tr_col, f32x16_t (&acc)[3]) {
  u32x4_t f[P::NR];
  f[0] = row_frag<TRI, SCH, P::ROW[0], KS>(S, l32, hi, tr_krow, tr_col);
  f[1] = row_frag<TRI, SCH, P::ROW[1], KS>(S, l32, hi, tr_krow, tr_col);
  if constexpr (P::NR > 2) f[2] = row_frag<TRI, SCH, P::ROW[2], KS>(S, l32, hi, tr_krow, tr_col);
#pragma unroll
  for (int k = 0; k < P::NTL; ++k) acc[k] = mfma(f[P::J[k]], f[P::I[k]], acc[k]);
}

template <class P, bool TRI, int SCH, int... KS>
HM_DEV void gram_steps(const lds_u8* S, int l32, int hi, int tr_krow, int tr_col, f32x16_t (&acc)[3],
                       std::integer_sequence<int, KS...>) {
  (gram_step<P, TRI, SCH, KS>(S, l32, hi, tr_krow, tr_col, acc), ...);
}

// acc[k] = (S S^T) tile k of wave W, S = LDS operand with SCH chunks per row
// and K = 8 SCH columns (TRI: a symmetric 128 x 128 matrix stored as its
// lower tiles). Lane holds element 4 q + e of acc[k] at
// C[32 ROW[I[k]] + l32][32 ROW[J[k]] + 8 q + 4 hi + e].
template <class P, bool TRI, int SCH>
HM_DEV void gram_mma(const lds_u8* S, int lane, f32x16_t (&acc)[3]) {
  const int ln = opaque_lane(lane), l32 = ln & 31, hi = ln >> 5;
  const int tr_krow = tr_krow_of(ln), tr_col = tr_col_of(ln);
#pragma unroll
  for (int k = 0; k < P::NTL; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[k][e] = 0.f;
  gram_steps<P, TRI, SCH>(S, l32, hi, tr_krow, tr_col, acc, std::make_integer_sequence<int, SCH / 2>{});
}

// Store wave W's bf16 tiles o[k][q] (q: 4 columns each) as lower tiles of
// the symmetric matrix C.
template <class P>
HM_DEV void gram_store(lds_u8* C, int lane, const u32x2_t (&o)[3][4]) {
  const int ln = opaque_lane(lane), l32 = ln & 31, hi = ln >> 5;
#pragma unroll
  for (int k = 0; k < P::NTL; ++k) {
    const int ti = P::ROW[P::I[k]], tj = P::ROW[P::J[k]];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<lds_u32x2*>(C + tri_pos(ti, tj, l32, q) + hi * 8) = o[k][q];
  }
}

// A = bf16(X X^T): wave W's tiles into A.
template <class P, int XCH>
HM_DEV void gram_a(const lds_u8* X, lds_u8* A, int lane) {
  f32x16_t acc[3];
  gram_mma<P, false, XCH>(X, lane, acc);
  u32x2_t o[3][4];
#pragma unroll
  for (int k = 0; k < P::NTL; ++k)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[k][q] = u32x2_t{pk_bf16(acc[k][4 * q], acc[k][4 * q + 1]), pk_bf16(acc[k][4 * q + 2], acc[k][4 * q + 3])};
  gram_store<P>(A, lane, o);
}

// B = bf16(c (A A^T) + b A) for wave W's tiles, into registers (A is still
// read by the other waves; the caller stores after a barrier).
template <class P>
HM_DEV void gram_b(const lds_u8* A, int lane, float cb, float cc, u32x2_t (&o)[3][4]) {
  constexpr int ACH = M / 8;
  f32x16_t acc[3];
  gram_mma<P, true, ACH>(A, lane, acc);
  const int ln = opaque_lane(lane), l32 = ln & 31, hi = ln >> 5;
#pragma unroll
  for (int k = 0; k < P::NTL; ++k) {
    const int ti = P::ROW[P::I[k]], tj = P::ROW[P::J[k]];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x2_t rv = *reinterpret_cast<lds_cu32x2*>(A + tri_pos(ti, tj, l32, q) + hi * 8);
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = fmaf(cb, bf16_to_f32(half16(rv[e >> 1], e & 1)), cc * acc[k][4 * q + e]);
      o[k][q] = u32x2_t{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
    }
  }
}

// B row-tile fragments R0 .. R0 + RT - 1 at k-step KS.
template <int R0, int KS, int... R>
HM_DEV void b_frags(const lds_u8* B, int l32, int hi, int tr_krow, int tr_col, u32x4_t (&fb)[sizeof...(R)],
                    std::integer_sequence<int, R...>) {
  ((fb[R] = tri_frag<R0 + R, KS>(B, l32, hi, tr_krow, tr_col)), ...);
}

// One k-step of Apply: acc[tj][ti] += X^T-column tile tj (transposing reads
// of X from column jb) times B row tile R0 + ti.
template <int TJ, int RT, int XCH, int R0, int KS>
HM_DEV void apply_step(const lds_u8* B, const lds_u8* X, int jb, int l32, int hi, int tr_krow, int tr_col,
                       f32x16_t (&acc)[TJ][RT]) {
  u32x4_t fb[RT], fa[TJ];
  b_frags<R0, KS>(B, l32, hi, tr_krow, tr_col, fb, std::make_integer_sequence<int, RT>{});
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj) {
    const int c0 = jb + 32 * tj + tr_col;
    const int kr = 16 * KS + tr_krow;
    const u32x2_t l2 = read_tr(X, lds_pos(kr, c0 >> 3, XCH) + (c0 & 7) * 2);
    const u32x2_t u2 = read_tr(X, lds_pos(kr + 4, c0 >> 3, XCH) + (c0 & 7) * 2);
    fa[tj] = u32x4_t{l2[0], l2[1], u2[0], u2[1]};
  }
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
    for (int ti = 0; ti < RT; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
}

template <int TJ, int RT, int XCH, int R0, int... KS>
HM_DEV void apply_steps(const lds_u8* B, const lds_u8* X, int jb, int lane, f32x16_t (&acc)[TJ][RT],
                        std::integer_sequence<int, KS...>) {
  const int ln = opaque_lane(lane), l32 = ln & 31, hi = ln >> 5;
  const int tr_krow = tr_krow_of(ln), tr_col = tr_col_of(ln);
  (apply_step<TJ, RT, XCH, R0, KS>(B, X, jb, l32, hi, tr_krow, tr_col, acc), ...);
}

// `steps` NS iterations on the tile X0 in LDS (X, 128 x 128 NQ), A/B in the
// lower-tile buffer A; X' replaces X. Every thread of the workgroup calls it;
// it ends with a workgroup barrier.
template <int NQ, int NW>
HM_DEV void ns_iterations(lds_u8* X, lds_u8* A, int lane, int steps, float ca, float cb, float cc,
                          int round_once) {
  constexpr int N = 128 * NQ;
  constexpr int XCH = N / 8;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar branches
  for (int it = 0; it < steps; ++it) {
    // ---- A = bf16(X X^T) ------------------------------------------------------
    with_part<NW>(wave, [&](auto part) { gram_a<decltype(part), XCH>(X, A, lane); });
    __syncthreads();

    // ---- B = bf16(c (A A^T) + b A), in place of A --------------------------------
    // (one dispatch on the wave-uniform index for the product, the barrier and
    // the store, so each wave's B tiles stay in registers across the barrier;
    // every wave reaches exactly one of the barriers)
    with_part<NW>(wave, [&](auto part) {
      u32x2_t o[3][4];
      gram_b<decltype(part)>(A, lane, cb, cc, o);
      __syncthreads();  // every read of A (products and the b A term) is done
      gram_store<decltype(part)>(A, lane, o);
    });
    __syncthreads();

    // ---- X' = bf16(bf16(B X) + a X), in place of X ------------------------------
    // Wave w owns columns w np/NW .. + np/NW - 1 over all 128 rows, in passes
    // of at most 64 columns. It reads only its own columns of X, so it
    // overwrites them as each pass ends, without waiting for the other waves.
    {
      constexpr int WCOL = N / NW;                // columns per wave
      constexpr int PT = WCOL >= 64 ? 2 : 1;      // 32-column tiles per pass
#pragma unroll 1
      for (int pass = 0; pass < WCOL / (32 * PT); ++pass) {
        const int jb = WCOL * wave + 32 * PT * pass;
        f32x16_t acc[PT][4];
#pragma unroll
        for (int a = 0; a < PT; ++a)
#pragma unroll
          for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;
        apply_steps<PT, 4, XCH, 0>(A, X, jb, lane, acc, std::make_integer_sequence<int, M / 16>{});
        const int ln = opaque_lane(lane), l32 = ln & 31, hi = ln >> 5;
        u32x2_t o[4][PT][4];
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
#pragma unroll
          for (int tj = 0; tj < PT; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int i = 32 * ti + l32;
              const int ch = (jb >> 3) + 4 * tj + q;
              const u32x2_t rv = *reinterpret_cast<lds_cu32x2*>(X + lds_pos(i, ch, XCH) + hi * 8);
              float y[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float v = acc[tj][ti][4 * q + e];
                const float bx = round_once ? v : bf16_to_f32(pk_bf16(v, 0.f) & 0xffffu);
                y[e] = fmaf(ca, bf16_to_f32(half16(rv[e >> 1], e & 1)), bx);
              }
              o[ti][tj][q] = u32x2_t{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
            }
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
#pragma unroll
          for (int tj = 0; tj < PT; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int i = 32 * ti + l32;
              const int ch = (jb >> 3) + 4 * tj + q;
              *reinterpret_cast<lds_u32x2*>(X + lds_pos(i, ch, XCH) + hi * 8) = o[ti][tj][q];
            }
      }
    }
    __syncthreads();
  }
}

// Threads per workgroup: 128 x 128 tiles run three 4-wave workgroups per CU;
// wider tiles (84 or 148 KiB of LDS, one workgroup per CU) run eight waves,
// two per SIMD.
template <int NQ>
constexpr int lds_threads() { return NQ == 1 ? NT : 2 * NT; }

template <int NQ, int NTQ = lds_threads<NQ>()>
__global__ __launch_bounds__(NTQ, NQ == 1 ? 3 : 1) void ns5_lds_kernel(const uint16_t* x,
                                                        uint16_t* out,
                                                        const float* __restrict__ inv,
                                                        int64_t ntiles, int steps, float ca,
                                                        float cb, float cc, int round_once) {
  constexpr int N = 128 * NQ;   // NS columns (np)
  constexpr int XCH = N / 8;    // 16-byte chunks per X row
  __shared__ __attribute__((aligned(16))) uint8_t sx_raw[M * N * 2];
  __shared__ __attribute__((aligned(16))) uint8_t sa_raw[TRI_BYTES];
  lds_u8* const X = (lds_u8*)sx_raw;
  lds_u8* const A = (lds_u8*)sa_raw;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;

  constexpr int VPT = M * XCH / NTQ;  // 16-byte chunks per thread
  // np = 256 (one workgroup per CU) loads the next tile during this tile's
  // iterations; np = 128 (three per CU, one tile per workgroup) leaves the
  // load latency to the other workgroups and keeps the registers; np = 512
  // has no registers to spare for a whole tile.
  constexpr bool PREFETCH = NQ == 2;
  u32x4_t v[VPT];
  auto load_tile = [&](int64_t t) {
    const uint16_t* src = x + t * (int64_t)M * N;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = k * NTQ + tid;
      v[k] = *reinterpret_cast<const u32x4_t*>(src + (int64_t)(idx / XCH) * N + (idx % XCH) * 8);
    }
  };
  if (PREFETCH && blockIdx.x < ntiles) load_tile(blockIdx.x);
  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    // ---- X0 = bf16(x * inv) into LDS ------------------------------------------
    const float sc = inv[t];
    if (!PREFETCH) load_tile(t);
    __syncthreads();  // the previous tile's final LDS reads are done
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = k * NTQ + tid;
      *reinterpret_cast<lds_u32x4*>(X + lds_pos(idx / XCH, idx % XCH, XCH)) = scale8(v[k], sc);
    }
    // the next tile's loads run under this tile's iterations
    if (PREFETCH && t + gridDim.x < ntiles) load_tile(t + gridDim.x);
    __syncthreads();

    ns_iterations<NQ, NTQ / 64>(X, A, lane, steps, ca, cb, cc, round_once);

    // ---- result -> global ----------------------------------------------------------
    uint16_t* dst = out + t * (int64_t)M * N;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = k * NTQ + tid;
      *reinterpret_cast<u32x4_t*>(dst + (int64_t)(idx / XCH) * N + (idx % XCH) * 8) =
          *reinterpret_cast<lds_cu32x4*>(X + lds_pos(idx / XCH, idx % XCH, XCH));
    }
  }
}

// The whole optimizer step of a bucket of 128 x 128 NS tiles in one launch
// (tile_h <= tile_w <= 128, so no transpose): per tile, the momentum update
// and gather (the gather kernel's arithmetic), the normaliser, the NS
// iterations and the untile with WD/LR (the fused untile's arithmetic), with
// the tile held in LDS from the momentum to the parameter update. HBM sees the
// grad, the momentum buffer (read and written) and the parameter (read and
// written) once each; no NS tile buffer exists. One tile per workgroup: the
// workgroups that start as others finish fall out of step with each other, so
// a CU's three workgroups are mostly in different phases (memory or NS). That
// measured faster than persistent workgroups that walk several tiles, even
// with one tile's untile and the next one's gather merged into one pass.
//
// Bit-identical to gather -> tile_scale -> NS5 -> untile_apply: every element
// is computed by the same per-element code, and the tile's sum of squares is
// accumulated in the gather kernel's order (256 threads; thread t sums the
// 8-element vectors t, t + 256, ..., t + 1792 of the 128 x 128 tile, each in
// element order; then the same wave and block reductions, and the same
// 1 / (sqrt(s) + eps)).
constexpr int SV_N = 128, SV_VPR = SV_N / 8;  // 16 vectors of 8 per NS row
constexpr int SV_VPT = M * SV_VPR / NT;       // vectors per thread (8)
// vectors loaded before any is used: the untile all 8 (8 VGPRs each), the
// gather 4 (16 VGPRs each; 8 would spill)
constexpr int SV_BATCH_UNT = 8, SV_BATCH_GAT = 4;

struct TileAt {
  const HimuonParamDesc* P;
  int r, c;
};

HM_DEV TileAt tile_at(const HimuonParamDesc* __restrict__ params, int n_params, int64_t t) {
  const HimuonParamDesc* P = params + find_param(params, n_params, t);
  const int64_t lt = t - P->tile0;
  return TileAt{P, (int)(lt / P->C), (int)(lt % P->C)};
}

// Exactly one of UNT and GAT. UNT: untile with WD/LR of tile tu from X (X'
// of the NS iterations). GAT: momentum and gather of tile tg into X (bf16(e),
// not yet normalised); returns this thread's sum of squares of it. Each
// thread reads and writes only its own vectors v = k NT + tid of X.
template <int DT, int PDT, bool UNT, bool GAT>
HM_DEV float step_io(const HimuonParamDesc* __restrict__ params, int n_params, lds_u8* X, int64_t tu, int64_t tg,
                     int tile_h, int tile_w, const float* __restrict__ sa) {
#pragma clang fp contract(off)
  static_assert(UNT != GAT, "one tile pass per call");
  constexpr int XCH = SV_N / 8;
  TileAt U{nullptr, 0, 0}, G{nullptr, 0, 0};
  float s = 0.f, alpha = 0.f, sc = 0.f, mu = 0.f;
  bool has_mom = false, nesterov = false;
  if constexpr (UNT) {
    U = tile_at(params, n_params, tu);
    s = sa[2 * U.P->group];
    alpha = sa[2 * U.P->group + 1];
    sc = U.P->upd_scale;
  }
  if constexpr (GAT) {
    G = tile_at(params, n_params, tg);
    has_mom = G.P->momentum != nullptr;
    mu = G.P->mu;
    nesterov = G.P->nesterov != 0;
  }
  // (addresses from an opaque copy of the thread index: shared with the other
  // pass and kept live across the NS iterations they would not fit beside
  // those iterations' registers)
  const int tq = opaque_lane((int)threadIdx.x);
  float ssq = 0.f;
  constexpr int SV_BATCH = UNT ? SV_BATCH_UNT : SV_BATCH_GAT;
#pragma unroll 1
  for (int b0 = 0; b0 < SV_VPT; b0 += SV_BATCH) {
    // phase 1: every global load of the batch (parameters of tile tu, or
    // grads and momentum of tile tg) before any is used
    float pv[SV_BATCH][8], g[SV_BATCH][8], m[SV_BATCH][8];
    bool uok[SV_BATCH], ufull[SV_BATCH], fast[SV_BATCH];
#pragma unroll
    for (int k = 0; k < SV_BATCH; ++k) {
      const int v = (b0 + k) * NT + tq;
      const int i = v / SV_VPR, j0 = (v % SV_VPR) * 8;
      if constexpr (UNT) {
        const int64_t pr = (int64_t)U.r * tile_h + i, pc = (int64_t)U.c * tile_w + j0;
        const int64_t ou = pr * U.P->ld_upd + pc;
        uok[k] = i < tile_h && j0 < tile_w && pr < U.P->h && pc < U.P->w;
        ufull[k] = uok[k] && j0 + 8 <= tile_w && pc + 8 <= U.P->w && aligned16<PDT>(U.P->update, ou);
        if (ufull[k]) load8<PDT>(U.P->update, ou, pv[k]);
      }
      if constexpr (GAT) {
        const int64_t pr = (int64_t)G.r * tile_h + i, pc = (int64_t)G.c * tile_w + j0;
        const int64_t og = pr * G.P->ld_grad + pc, om = pr * G.P->ld_mom + pc;
        fast[k] = i < tile_h && pr < G.P->h && j0 + 8 <= tile_w && pc + 8 <= G.P->w &&
                  aligned16<DT>(G.P->grad, og) && (!has_mom || aligned16<DT>(G.P->momentum, om));
        if (fast[k]) {
          load8<DT>(G.P->grad, og, g[k]);
          if (has_mom) load8<DT>(G.P->momentum, om, m[k]);
        }
      }
    }
    // phase 2: the untile reads X' of vector v, or the gather writes it
#pragma unroll
    for (int k = 0; k < SV_BATCH; ++k) {
      const int v = (b0 + k) * NT + tq;
      const int i = v / SV_VPR, j0 = (v % SV_VPR) * 8;
      lds_u32x4* const px = reinterpret_cast<lds_u32x4*>(X + lds_pos(i, v % SV_VPR, XCH));
      if constexpr (UNT) {
        if (uok[k]) {
          const u32x4_t w = *px;
          float y[8];
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            y[2 * e2] = sc * bf16_to_f32(w[e2] & 0xffffu);
            y[2 * e2 + 1] = sc * __uint_as_float(w[e2] & 0xffff0000u);
          }
          const int64_t pr = (int64_t)U.r * tile_h + i, pc = (int64_t)U.c * tile_w + j0;
          const int64_t ou = pr * U.P->ld_upd + pc;
          if (ufull[k]) {  // put8<true>'s full form, its load issued above
#pragma unroll
            for (int e = 0; e < 8; ++e)
              pv[k][e] = __builtin_fmaf(alpha, round_to<PDT>(y[e]), round_to<PDT>(pv[k][e] * s));
            store8<PDT>(U.P->update, ou, pv[k]);
          } else {
            const int valid = (int)min<int64_t>(min(8, tile_w - j0), U.P->w - pc);
            put8<true, PDT>(*U.P, ou, y, false, valid, sa);
          }
        }
      }
      if constexpr (GAT) {
        const int64_t pr = (int64_t)G.r * tile_h + i, pc = (int64_t)G.c * tile_w + j0;
        const int64_t og = pr * G.P->ld_grad + pc, om = pr * G.P->ld_mom + pc;
        float x[8];
        if (fast[k]) {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = momentum_elem<DT>(g[k][e], &m[k][e], mu, nesterov, has_mom);
          if (has_mom) store8<DT>(G.P->momentum, om, m[k]);
        } else {
          const bool row_ok = i < tile_h && pr < G.P->h;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            x[e] = 0.f;
            if (row_ok && j0 + e < tile_w && pc + e < G.P->w) {
              const float gv = load_elem<DT>(G.P->grad, og + e);
              float mv = has_mom ? load_elem<DT>(G.P->momentum, om + e) : 0.f;
              x[e] = momentum_elem<DT>(gv, &mv, mu, nesterov, has_mom);
              if (has_mom) store_elem<DT>(G.P->momentum, om + e, mv);
            }
          }
        }
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          h[e] = f32_to_bf16(x[e]);
          const float f = bf16_to_f32(h[e]);
          ssq = fmaf(f, f, ssq);
        }
        *px = u32x4_t{pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7])};
      }
    }
  }
  return ssq;
}

template <int DT, int PDT>
__global__ __launch_bounds__(NT, 3) void lds_step_kernel(const HimuonParamDesc* __restrict__ params, int n_params,
                                                         int64_t tile_begin, int64_t ntiles, int tile_h,
                                                         int tile_w, int steps, float ca, float cb, float cc,
                                                         float eps, int round_once,
                                                         const float* __restrict__ sa) {
  constexpr int XCH = SV_N / 8;
  __shared__ __attribute__((aligned(16))) uint8_t sx_raw[M * SV_N * 2];
  __shared__ __attribute__((aligned(16))) uint8_t sa_raw[TRI_BYTES];
  __shared__ float red[NT / 64];
  __shared__ float s_inv;
  lds_u8* const X = (lds_u8*)sx_raw;
  lds_u8* const A = (lds_u8*)sa_raw;
  const int lane = threadIdx.x & 63;

  const int64_t tt = blockIdx.x;  // the grid has one workgroup per tile
  if (tt >= ntiles) return;
  const float ssq = step_io<DT, PDT, false, true>(params, n_params, X, 0, tile_begin + tt, tile_h, tile_w, sa);
  // ---- normaliser (the gather's block sum, then tile_scale), X0 in place ----------
  const float sum = block_sum<NT>(ssq, red);
  if (threadIdx.x == 0) s_inv = 1.0f / (sqrtf(0.f + sum) + eps);
  __syncthreads();
  const float inv = s_inv;
  const int ts = opaque_lane((int)threadIdx.x);
#pragma unroll
  for (int k = 0; k < SV_VPT; ++k) {
    const int v = k * NT + ts;
    lds_u32x4* const px = reinterpret_cast<lds_u32x4*>(X + lds_pos(v / SV_VPR, v % SV_VPR, XCH));
    *px = scale8(*px, inv);
  }
  __syncthreads();

  ns_iterations<1, 4>(X, A, lane, steps, ca, cb, cc, round_once);

  // ---- untile with WD/LR ----------------------------------------------------------
  step_io<DT, PDT, true, false>(params, n_params, X, tile_begin + tt, 0, tile_h, tile_w, sa);
}

int num_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

}  // namespace

bool lds_step_supported(int tile_h, int tile_w, int dtype, int param_dtype) {
  return tile_h > 0 && tile_h <= tile_w && tile_w <= M &&
         (dtype == HIMUON_DTYPE_F32 || dtype == HIMUON_DTYPE_BF16) &&
         (param_dtype == HIMUON_DTYPE_F32 || param_dtype == HIMUON_DTYPE_BF16);
}

void lds_step_run(const HimuonParamDesc* params, int n_params, int64_t tile_begin, int64_t cnt, int tile_h,
                  int tile_w, int dtype, int param_dtype, int steps, float a, float b, float c, float eps,
                  bool round_once, const float* sa, hipStream_t s) {
  // one workgroup per tile, in launches of at most 2^30 workgroups
  const int ro = round_once ? 1 : 0;
  const dim3 block(NT);
  for (int64_t off = 0; off < cnt; off += (int64_t)1 << 30) {
    const int64_t n = std::min<int64_t>(cnt - off, (int64_t)1 << 30);
    const dim3 grid((unsigned)n);
#define HM_LDS_STEP(D, PD)                                                                                    \
  hipLaunchKernelGGL((lds_step_kernel<D, PD>), grid, block, 0, s, params, n_params, tile_begin + off, n, tile_h, \
                     tile_w, steps, a, b, c, eps, ro, sa)
    if (dtype == HIMUON_DTYPE_F32) {
      if (param_dtype == HIMUON_DTYPE_F32) HM_LDS_STEP(HIMUON_DTYPE_F32, HIMUON_DTYPE_F32);
      else HM_LDS_STEP(HIMUON_DTYPE_F32, HIMUON_DTYPE_BF16);
    } else {
      if (param_dtype == HIMUON_DTYPE_F32) HM_LDS_STEP(HIMUON_DTYPE_BF16, HIMUON_DTYPE_F32);
      else HM_LDS_STEP(HIMUON_DTYPE_BF16, HIMUON_DTYPE_BF16);
    }
  }
#undef HM_LDS_STEP
}

bool ns5_lds_supported(int mp, int np) { return mp == M && (np == 128 || np == 256 || np == 512); }

void ns5_lds_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                 float a, float b, float c, bool round_once, hipStream_t s) {
  (void)mp;
  uint16_t* out = (steps & 1) ? y : x;
  // np = 128: one workgroup per tile (up to 2^30 per launch; the kernel's tile
  // loop takes the rest), 4 % faster than persistent workgroups; wider tiles:
  // persistent, prefetching the next tile (np = 256)
  const int64_t wgs = np == 128 ? std::min<int64_t>(cnt, (int64_t)1 << 30)
                                : std::min<int64_t>(cnt, (int64_t)4 * num_cus());
  if (np == 128)
    hipLaunchKernelGGL(ns5_lds_kernel<1>, dim3((unsigned)wgs), dim3(lds_threads<1>()), 0, s, x, out, inv, cnt, steps, a, b, c, round_once ? 1 : 0);
  else if (np == 256)
    hipLaunchKernelGGL(ns5_lds_kernel<2>, dim3((unsigned)wgs), dim3(lds_threads<2>()), 0, s, x, out, inv, cnt, steps, a, b, c, round_once ? 1 : 0);
  else
    hipLaunchKernelGGL(ns5_lds_kernel<4>, dim3((unsigned)wgs), dim3(lds_threads<4>()), 0, s, x, out, inv, cnt, steps, a, b, c, round_once ? 1 : 0);
}
