// Fused second and third NS products for 512 x 512 NS tiles ("BA" kernel):
//
//   B  = bf16(c A A^T + b A)                  (ba_plus_cAA.py:58-85)
//   X' = bf16(bf16(B X) + a X)                (fused_bmm_add.py:65-88)
//        bf16(B X + a X) with round_once      (torch.addmm, himuon.py:249-253)
//
// one 128-row panel of one tile per work item, so that B never leaves the
// CU: per tile and iteration HBM carries A and X in and X' out (1.5 MiB)
// instead of A in, B out, B and X in and X' out (2.5 MiB). The first product
// (A = bf16(X X^T)) stays the streamed Gram kernel (ns5_stream.hip).
//
// Work item (tile t, panel p), rows i0 = 128 p .. i0 + 127, eight waves, two
// per SIMD: wave w = 4 h + c (group h, SIMD c) owns output columns
// col0 = 256 h + 64 c .. + 63 in both stages, as 2 x 4
// v_mfma_f32_32x32x16_bf16 tiles (128 fp32 accumulators per lane). Items are
// spread persistently, a contiguous range per XCD.
//
//  Stage 1: B_P[i][j] = bf16(c sum_k A[i0+i][k] A[j][k] + b A[i0+i][j]).
//    Row-side operand A_P (128 x 512 bf16 = 128 KiB) resident in LDS region
//    R. Column-side operand: A is exactly symmetric, so A[j][k] = A[k][j]
//    and the wave streams rows k of A restricted to its 64 columns.
//  Stage 2: X'_P[i][j] = bf16(bf16(sum_k B_P[i][k] X[k][j]) + a X[i0+i][j]).
//    Row-side operand B_P, written over A_P in R by the stage-1 epilogue;
//    column-side operand: rows k of X restricted to the wave's columns.
//
// Each wave runs six phases per item, each ended by a workgroup barrier:
//   K1a, K1b  stage-1 K loop over k = 0..255, then k = 256..511
//   E1        stage-1 epilogue: B_P = bf16(c acc + b A_P) over the wave's
//             own 128 x 64 block column of A_P (block column 4 h + c)
//   K2a, K2b  stage-2 K loop, the same two halves
//   E2        stage-2 epilogue: + a X_P, stores of X'_P; direct-to-LDS load
//             of the next item's A_P half h (block columns 4 h .. 4 h + 3)
// Group 1 (waves 4..7) passes one extra barrier first, so it runs one phase
// behind group 0 (waves 0..3): on every SIMD one wave's epilogue meets the
// other wave's K loop, and the MFMA pipe has work while either epilogue runs.
// Barrier segment s holds phase s of group 0 and phase s - 1 of group 1:
//   K1a | E2(prev)    K1b | K1a    E1 | K1b    K2a | E1    K2b | K2a    E2 | K2b
// which orders every LDS reuse of R:
//  - E1 of group 0 (segment 3) overwrites A_P block columns 0..3, whose last
//    readers are the K1a halves (segments 1, 2); E1 of group 1 (segment 4)
//    block columns 4..7, last read in the K1b halves (segments 2, 3);
//  - K2a (block columns 0..3 of B_P) starts after E1 of group 0, K2b (4..7)
//    after E1 of group 1;
//  - E2 of group 0 (segment 6) loads the next A_P's columns 0..3 after both
//    K2a halves (segments 4, 5) and waits for them before its barrier, for
//    the next K1a of group 0 (next segment 1); E2 of group 1 (next segment 1)
//    loads columns 4..7 after both K2b halves (segments 5, 6), landed before
//    the next K1b of group 0 (next segment 2).
// Within a K-loop half the R fragments of the next k-step are read one k-step
// ahead, but never across the half boundary (the other half of R may still be
// written in that segment).
//
//  K loops: the streamed rows go from global memory into a four-unit register
//  ring (a unit = 32 rows x 64 columns = two k-steps of 16, 4 x 16-byte loads
//  per lane); each k-step's 16 rows are written to one of two wave-private
//  2 KiB staging buffers one unit before its MFMAs and read back as column
//  fragments with ds_read_b64_tr_b16 (contraction along the rows). A slot is
//  free once its rows are staged, so it takes the unit four ahead while the
//  staged unit's MFMAs run: loads are issued three units before the rows are
//  staged.
//  After stage 2 the ring carries the X_P rows i0 .. i0 + 127 (the a X term).
//
//  Stage-2 epilogue, per 32-row block: bf16(B X) through the wave's 4 KiB
//  area into the row layout of the stores, + a X there with the X_P rows the
//  ring holds in that layout, 128-byte row stores, and the next item's first
//  ring units loaded. (The 2-D form rounds B X + a X once: X_P goes into the
//  accumulator layout through the area instead, and the sum back.)
//
// Each output element sums its k terms in one fp32 accumulator in ascending k
// with the same MFMA as the three-kernel path, so results are bit-identical
// to it.
//
// LDS: R (128 KiB, 8-row blocks, below), then a 4 KiB area per wave: two
// 2 KiB staging buffers (16 rows x 128 B, 16-byte chunk c of row r at
// c ^ 4 ((r / 2) % 2), conflict-free for the row writes and the transposing
// reads); in the epilogue one block of 32 rows x 128 B, chunk c of row r at
// c ^ (r / 2) % 8.
#include "elem_ops.h"
#include "ns5_kernels.h"

namespace {

constexpr int T = 512;           // tile edge (mp = np)
constexpr int P = 128;           // panel rows
constexpr int NW = 8;            // waves, two per SIMD
constexpr int NTH = 64 * NW;
constexpr int R_BYTES = P * T * 2;          // 128 KiB
constexpr int WAREA = 4096;                 // per-wave staging
constexpr int LDS_BYTES = R_BYTES + NW * WAREA;
constexpr int NKS = T / 16;                 // k-steps per stage
constexpr int NUNIT = T / 32;               // ring units per stage (2 k-steps each)
constexpr int HUNIT = NUNIT / 2;            // ring units per K-loop half
constexpr int NSLOT = 4;                    // ring slots
// units in flight: a unit's rows are staged one unit before its MFMAs, so
// its slot takes the unit NSLOT ahead while those MFMAs run
constexpr int AHEAD = NSLOT;
static_assert(LDS_BYTES == 160 * 1024, "LDS budget");

struct BaArgs {
  const uint16_t* A;   // (ntiles, T, T) bf16, symmetric
  const uint16_t* X;   // (ntiles, T, T) bf16
  uint16_t* Y;         // (ntiles, T, T) bf16 output X'
  int64_t ntiles;
  float a, b, c;
  int round_once;
  const float* xinv;   // SC: X is the raw tile, X0 = bf16(X xinv[tile]) used in its place
  BaUntile u;          // the fused untile of the last iteration (kernels with UDT >= 0)
};

typedef __attribute__((address_space(3))) u32x4_t lds_u32x4;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

HM_DEV u32x2_t read_tr(const lds_u8* p) {
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)p);
  return __builtin_bit_cast(u32x2_t, r);
}

// 16 bytes at a wave-uniform base plus a 32-bit byte offset (the
// scalar-base + vector-offset form of the load: no 64-bit address per lane).
HM_DEV u32x4_t gload16(const uint16_t* base, uint32_t off) {
  return *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(base) + off);
}
// Non-temporal store (nt): X' is not read again by this launch, so its lines
// should not displace the A and X rows the tile's other panels still stream
// from L2 (reads 1.5x -> 1.34x the unique A and X per 4,096-tile launch).
HM_DEV void gstore16(uint16_t* base, uint32_t off, u32x4_t v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(reinterpret_cast<char*>(base) + off));
}

// ---- the fused untile of the last NS iteration (kernels with UDT >= 0) -------------
// Per-tile record of the launch's tiles, written by untile_rec_kernel before
// the fused kernel runs (16 int32 per tile, the parameter's descriptor found
// once per tile instead of once per work item and wave):
//   0-1 parameter base  2-3 row stride  4-5 rows h  6-7 columns w
//   8-9 parameter row of the tile's (0, 0)  10-11 its column  12 upd_scale bits  13 group
constexpr int kRecInts = 16;
static_assert(2 * HIMUON_APPLY_MAX_GROUPS == 64, "one (scale, alpha) value per lane");

__global__ void untile_rec_kernel(BaUntile u, int64_t cnt) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= cnt) return;
  const int64_t bt = u.tile0 + t;
  const HimuonParamDesc& P = u.params[find_param(u.params, u.n_params, bt)];
  const int64_t lt = bt - P.tile0;
  const int64_t v[6] = {(int64_t)(uintptr_t)P.update, P.ld_upd, P.h, P.w, (lt / P.C) * u.tile_h, (lt % P.C) * u.tile_w};
  int32_t* r = u.rec + t * kRecInts;
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    r[2 * k] = (int32_t)(uint32_t)(uint64_t)v[k];
    r[2 * k + 1] = (int32_t)(uint32_t)((uint64_t)v[k] >> 32);
  }
  r[12] = __float_as_int(P.upd_scale);
  r[13] = P.group;
  r[14] = r[15] = 0;
}

struct UParam {
  void* base;        // the parameter (its descriptor's `update`)
  int64_t h, w, ld;  // shape and row stride
  int64_t r0, c0;    // parameter row and column of the tile's element (0, 0)
  float sc;          // upd_scale
  float s, alpha;    // the group's (1 - lr wd, -lr)
};

// A tile's record (lane k < 16 holds int k, loaded at the item's start) and
// the (scale, alpha) table (lane k holds float k) as wave-uniform values.
HM_DEV UParam uparam_get(int recv, float sav) {
  auto rd = [&](int k) { return (uint32_t)__builtin_amdgcn_readlane(recv, k); };
  auto i64 = [&](int k) { return (int64_t)(((uint64_t)rd(k + 1) << 32) | rd(k)); };
  UParam p;
  p.base = (void*)(uintptr_t)i64(0);
  p.ld = i64(2);
  p.h = i64(4);
  p.w = i64(6);
  p.r0 = i64(8);
  p.c0 = i64(10);
  p.sc = __uint_as_float(rd(12));
  const int group = (int)rd(13);
  p.s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sav), 2 * group));
  p.alpha = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sav), 2 * group + 1));
  return p;
}

// Parameter accesses of the fused untile go through global-address-space
// pointers: as flat accesses (what a pointer read from a record becomes) they
// would also count in lgkmcnt, and every LDS wait of the epilogue would then
// wait for the parameter loads and stores in flight.
typedef __attribute__((address_space(1))) u32x4_t g_u32x4;
typedef __attribute__((address_space(1))) uint16_t g_u16;
typedef __attribute__((address_space(1))) float g_f32;

// One 32-row block of X' as the untile with WD/LR of himuon_untile_apply
// applies it (elem_ops.h put8 / wdlr8 / wdlr_elems): lane rows[n] holds tile
// row i + 8 n, columns j .. j + 7 (bf16); u = upd_scale X' (fp32), and
// p = rd(fma(alpha, rd(u), rd(p s))) for every element inside the tile and the
// parameter. Whole 8-element vectors load their parameter values first (all
// 4 rows, 2 at a time for fp32 parameters); others go one element at a time.
// u = upd_scale X' for the 8 bf16 values of x.
HM_DEV void ba_updates(const u32x4_t x, float sc, float (&y)[8]) {
#pragma unroll
  for (int w2 = 0; w2 < 4; ++w2) {
    y[2 * w2] = sc * __uint_as_float(x[w2] << 16);
    y[2 * w2 + 1] = sc * __uint_as_float(x[w2] & 0xffff0000u);
  }
}

// 8 parameter values as load8<DT> reads them, from their raw bytes.
template <int DT>
HM_DEV void ba_unpack(const u32x4_t (&raw)[DT == HIMUON_DTYPE_F32 ? 2 : 1], float (&p)[8]) {
#pragma unroll
  for (int w2 = 0; w2 < 4; ++w2) {
    if constexpr (DT == HIMUON_DTYPE_F32) {
      p[w2] = __uint_as_float(raw[0][w2]);
      p[4 + w2] = __uint_as_float(raw[1][w2]);
    } else {
      p[2 * w2] = bf16_to_f32(raw[0][w2] & 0xffffu);
      p[2 * w2 + 1] = __uint_as_float(raw[0][w2] & 0xffff0000u);
    }
  }
}

// 8 parameter values stored as store8<DT> stores them.
template <int DT>
HM_DEV void ba_store(g_u32x4* dst, const float (&p)[8]) {
  if constexpr (DT == HIMUON_DTYPE_F32) {
    __builtin_nontemporal_store(
        u32x4_t{__float_as_uint(p[0]), __float_as_uint(p[1]), __float_as_uint(p[2]), __float_as_uint(p[3])}, dst);
    __builtin_nontemporal_store(
        u32x4_t{__float_as_uint(p[4]), __float_as_uint(p[5]), __float_as_uint(p[6]), __float_as_uint(p[7])}, dst + 1);
  } else {
    u32x4_t w;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) w[w2] = pack2(f32_to_bf16(p[2 * w2]), f32_to_bf16(p[2 * w2 + 1]));
    __builtin_nontemporal_store(w, dst);
  }
}

// make_rows(rows) produces the block's X' rows (its LDS staging); EARLY: the
// whole-vector path issues its first parameter loads before calling it, so
// that their latency overlaps the staging (the loads' registers are then
// live beside the staging's). Returns whether the block took the
// whole-vector path (wave-uniform): its VMEM instructions are then 4 NQ loads
// and 4 NQ stores; on the element path their number depends on the data and
// may be zero.
template <int DT, bool EARLY, typename MakeRows>
HM_DEV bool ba_untile_block(const UParam& up, const BaUntile& u, MakeRows&& make_rows, int i, int j) {
#pragma clang fp contract(off)
  static_assert(DT == HIMUON_DTYPE_F32 || DT == HIMUON_DTYPE_BF16, "fp32 or bf16 parameters");
  constexpr bool F32 = DT == HIMUON_DTYPE_F32;
  constexpr int ES = F32 ? 4 : 2, NQ = F32 ? 2 : 1;
  u32x4_t rows[4];
  if constexpr (!EARLY) make_rows(rows);
  const int64_t pc = up.c0 + j;
  const bool col_ok = j < u.tile_w && pc < up.w;
  const bool col_full = j + 8 <= u.tile_w && pc + 8 <= up.w;
  char* const base = static_cast<char*>(up.base);
  const int64_t ou0 = (up.r0 + i) * up.ld + pc;  // row i's first element
  // The common case, decided per wave (no divergent branch, so the compiler
  // counts the loads in flight exactly instead of waiting for all of them):
  // every lane's 4 rows are whole, 16-byte aligned 8-element vectors.
  const bool all_full = col_full && i + 24 < u.tile_h && up.r0 + i + 24 < up.h &&
                        aligned16<DT>(up.base, ou0) && ((up.ld * ES) & 15) == 0;
  if (__all(all_full)) {
    constexpr int NB = F32 ? 2 : 4;  // rows whose loads are in flight together
#pragma unroll
    for (int n0 = 0; n0 < 4; n0 += NB) {
      u32x4_t raw[NB][NQ];
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const g_u32x4* src = (const g_u32x4*)(base + (ou0 + 8 * (n0 + k) * up.ld) * ES);
#pragma unroll
        for (int q = 0; q < NQ; ++q) raw[k][q] = __builtin_nontemporal_load(src + q);
      }
      if (EARLY && n0 == 0) make_rows(rows);
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        float y[8], p[8];
        ba_updates(rows[n0 + k], up.sc, y);
        ba_unpack<DT>(raw[k], p);
        wdlr8<DT>(p, y, up.s, up.alpha);
        ba_store<DT>((g_u32x4*)(base + (ou0 + 8 * (n0 + k) * up.ld) * ES), p);
      }
    }
    return true;
  }
  // Edge tiles, ragged or unaligned parameters: element by element inside
  // the tile and the parameter, as wdlr_elems<DT> (static indices).
  if constexpr (EARLY) make_rows(rows);
  const int valid = col_ok ? (int)min<int64_t>(min(8, u.tile_w - j), up.w - pc) : 0;
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int ii = i + 8 * n;
    const int64_t pr = up.r0 + ii;
    const int nv = (ii < u.tile_h && pr < up.h) ? valid : 0;
    if (nv == 0) continue;
    const int64_t ou = pr * up.ld + pc;
    float y[8];
    ba_updates(rows[n], up.sc, y);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (e < nv) {
        if constexpr (F32) {
          g_f32* q = (g_f32*)(base + (ou + e) * ES);
          const float p1 = round_to<DT>(*q * up.s);
          *q = __builtin_fmaf(up.alpha, round_to<DT>(y[e]), p1);
        } else {
          g_u16* q = (g_u16*)(base + (ou + e) * ES);
          const float p1 = round_to<DT>(bf16_to_f32(*q) * up.s);
          *q = (uint16_t)f32_to_bf16(__builtin_fmaf(up.alpha, round_to<DT>(y[e]), p1));
        }
      }
    }
  }
  return false;
}

// One ring unit: 4 x 16 bytes per lane (32 rows x 64 columns per wave).
struct Unit {
  u32x4_t v[4];
};

// Region R holds a 128 x 512 panel (A_P, then B_P) in 1 KiB blocks of 8 rows
// x 64 k: block (g, m) (rows 8 g .., k = 64 m ..) at (8 g + m) KiB, row r % 8
// at 128 (r % 8), 16-byte chunk c (k = 64 m + 8 c ..) at position
// c ^ swz(r). One direct-to-LDS instruction fills a block from 8 rows x 128
// contiguous bytes; the 16 lanes of a fragment read (rows r .. r + 15, one
// chunk) hit 16 distinct 16-byte bank groups.
HM_DEV int r_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// VMEM instructions a stage-2 epilogue issues after its direct-to-LDS loads
// (at its third 32-row block) when another item follows: 2 x 4 row stores
// and 2 x 4 ring loads (blocks 2, 3). The wait for those loads allows this
// many younger ones outstanding (vmcnt retires in issue order); the ring
// loads alone are E2_RING_AFTER_DMA. (Issued at the second block, the loads
// fetched 9 % more from HBM per launch in the same time: the next panel's
// lines had more time to leave L2 before the tile's streams passed them.)
constexpr int E2_RING_AFTER_DMA = 2 * 4;
constexpr int E2_VMEM_AFTER_DMA = 2 * 4 + E2_RING_AFTER_DMA;
static_assert(E2_VMEM_AFTER_DMA < 64, "vmcnt range");

// SC (the first iteration): every X value (stage-2 rows, the a X term) is
// replaced by bf16(x xinv[tile]) before it is used. UDT >= 0 (the last
// iteration of himuon_ns5_untile_apply, not SC): X' is not stored; the
// untile with WD/LR applies it to the parameters (dtype UDT) of g.u.
template <bool ROUND_ONCE, bool SC, int UDT = -1>
__global__ __launch_bounds__(NTH, 1) void ns_ba_kernel(BaArgs g) {
  static_assert(UDT < 0 || !SC, "the fused untile runs in a last iteration that is not the first");
  __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[LDS_BYTES];
  lds_u8* const lds = (lds_u8*)lds_raw;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, cw = wave & 3;
  const int col0 = 256 * grp + 64 * cw;  // the wave's first output column
  const int l32 = lane & 31, hi = lane >> 5;
  const uint32_t r_base = (uint32_t)(uintptr_t)lds;
  // R row fragments: fragment (ti, ks) of lane l (row 32 ti + l32, chunk
  // 2 (ks % 4) + hi of block column ks / 4) is at a per-k-step lane base
  // plus the immediate 32 KiB ti. The chunk term is made opaque per k-step,
  // so that the bases are formed where they are used (two VALU operations)
  // instead of being held through the K loops.
  const int rl_row = 8192 * (l32 >> 3) + 128 * (l32 & 7);
  const int rl_sw = hi ^ r_swz(l32);
  auto rfrag_base = [&](int ks) -> const lds_u8* {
    int sw = rl_sw;
    asm volatile("" : "+v"(sw));
    return lds + rl_row + 16 * ((2 * (ks & 3)) ^ sw) + 1024 * (ks >> 2);
  };
  lds_u8* const W = lds + R_BYTES + wave * WAREA;
  // Row writes: lane l writes row 8 n + l / 8 (n = 0, 1), chunk l % 8.
  const int wr = lane >> 3;
  lds_u8* const xw = W + 128 * wr + (((lane & 7) ^ (4 * ((wr >> 1) & 1))) << 4);
  // Transposing reads, 16-lane group i = l % 16: rows 8 hi + i / 4 (+ 4 for
  // the upper four k), bytes 32 ((l / 16) % 2) + 8 (i % 4) of the tile's
  // 64-byte segment, which sits at segment t2 ^ (i / 8) % 2 of the row.
  const int tr_i = lane & 15;
  const lds_u8* const xr0 = W + 128 * (8 * hi + (tr_i >> 2)) + 32 * ((lane >> 4) & 1) + 8 * (lane & 3);
  const int tr_s = (tr_i >> 3) & 1;
  // epilogue block (32 rows x 128 B, chunk c of row r at c ^ (r / 2) % 8)
  auto ep_off = [](int row, int chunk) { return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4); };

  // (32-bit item indices: the launcher takes at most kBaMaxTiles tiles per call)
  const int total = (int)g.ntiles * (T / P);
  const int wper = (int)(gridDim.x >> 3);
  const int per_xcd = (total + 7) >> 3;
  const int ibeg = (int)(blockIdx.x & 7) * per_xcd;
  const int iend = (ibeg + per_xcd < total) ? ibeg + per_xcd : total;
  int item = ibeg + (int)(blockIdx.x >> 3);
  if (item >= iend) return;

  // Unit of 32 rows restricted to the wave's 64 columns: lane l holds row
  // row0 + 8 n + l / 8, columns col0 + 8 (l % 8) .. + 7, in v[n].
  const uint32_t x_lane = 2u * ((lane >> 3) * T + col0 + 8 * (lane & 7));
  auto load_row = [&](const uint16_t* M, int row0, Unit& d, int n) { d.v[n] = gload16(M + (row0 + 8 * n) * T, x_lane); };
  auto load_rows = [&](const uint16_t* M, int row0, Unit& d) {
#pragma unroll
    for (int n = 0; n < 4; ++n) load_row(M, row0, d, n);
  };
  // Half hh of A_P (block columns m = 4 hh .. 4 hh + 3, k = 256 hh ..) into
  // R, one block per instruction: lane l lands at row l / 8, position l % 8
  // and fetches chunk (l % 8) ^ swz(row); the wave of SIMD wv takes block
  // rows 4 wv .. 4 wv + 3 (ln, wv: the lane and SIMD index, opaque per call
  // so the addresses are formed where they are used). 16 instructions.
  auto dma_half = [&](const uint16_t* At, int i0, int hh, int ln, int wv) {
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      const int gb = 4 * wv + gg;
      const int rr = ln >> 3;
      const int ch = (ln & 7) ^ rr ^ (gg & 1);
      const uint16_t* src = At + (i0 + 8 * gb + rr) * T + 256 * hh + 8 * ch;
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) dma16(src + 64 * mm, r_base + 1024 * (8 * gb + 4 * hh + mm));
    }
  };

  Unit ring[NSLOT];
  {
    // the first item's whole A_P (each group its half) and stage-1 units
    const uint16_t* At = g.A + (item >> 2) * (int64_t)T * T;
    dma_half(At, P * (int)(item & 3), grp, lane, cw);
#pragma unroll
    for (int u = 0; u < AHEAD; ++u) load_rows(At, 32 * u, ring[u]);
    wait_vm<AHEAD * 4>();
    lds_barrier();
  }
  const float ca = g.a, cb = g.b, cc = g.c;
  // group 1 runs one phase behind group 0: its first segment is empty
  if (grp == 1) lds_barrier();

  for (;;) {
    // The lane index, opaque per item: lane-dependent addresses are formed
    // inside the item loop, not hoisted out of it for the whole kernel (they
    // would not fit in the registers left beside the ring and accumulators).
    // (read by volatile assembly: a pure builtin would be hoisted and held.)
    int lane_o, cw_o = cw;
    uint32_t xl_o = x_lane;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_o));
    asm volatile("" : "+s"(cw_o), "+v"(xl_o));
    const int64_t tile = item >> 2;
    const int i0 = P * (int)(item & 3);
    const uint16_t* At = g.A + tile * (int64_t)T * T;
    const uint16_t* Xt = g.X + tile * (int64_t)T * T;
    uint16_t* Yt = g.Y + tile * (int64_t)T * T;
    const int next = item + wper;
    const bool more = next < iend;
    const uint16_t* const nAt = g.A + ((more ? next : item) >> 2) * (int64_t)T * T;
    const int ni0 = P * (next & 3);
    float xs = 1.f;
    if constexpr (SC) xs = uniform_load_f32(g.xinv, tile);
    // fused untile: the tile's record and the (scale, alpha) table, one int
    // or float per lane, first used in the stage-2 epilogue
    int urec = 0;
    float usa = 0.f;
    if constexpr (UDT >= 0) {
      typedef __attribute__((address_space(1))) const int32_t g_ci32;
      typedef __attribute__((address_space(1))) const float g_cf32;
      urec = lane < kRecInts ? ((g_ci32*)g.u.rec)[tile * kRecInts + lane] : 0;
      usa = ((g_cf32*)g.u.sa)[lane];
    }

    f32x16_t acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

    // ---- one K-loop half: acc += P_frag x (rows of M), k = 256 hf .. + 255 ----------
    // k-step ks: its 16 rows (ring unit ks / 2, registers 2 (ks % 2) ..) go to
    // staging buffer ks % 2 and come back as column fragments through
    // transposing reads; the row fragments of the panel (A_P or B_P) come from
    // R. One register set per fragment, refilled for k-step ks + 1 (within the
    // half) right after its last MFMA of k-step ks: the column fragment of
    // row 0 after that row, each row fragment after its MFMA in row 1, the
    // column fragment of row 1 after it; then k-step ks + 2's rows into
    // buffer ks % 2, behind those reads (a wave's LDS operations execute in
    // order). After each row, one load of the unit four ahead (into the slot
    // of unit u, whose rows were staged during unit u - 1).
    u32x4_t fa[2], fb[4];
    auto read_fa = [&](int ks, int t2) {
      const lds_u8* p = xr0 + 2048 * (ks & 1) + ((t2 ^ tr_s) << 6);
      const u32x2_t lo = read_tr(p);
      const u32x2_t up = read_tr(p + 512);
      fa[t2] = u32x4_t{lo[0], lo[1], up[0], up[1]};
    };
    auto write_rows = [&](int ks, const Unit& su, bool xrows) {
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        u32x4_t v = su.v[2 * (ks & 1) + n];
        if (SC && xrows) v = scale8_rne(v, xs);
        *reinterpret_cast<lds_u32x4*>(xw + 2048 * (ks & 1) + 1024 * n) = v;
      }
    };
    // stream unit v of this item: stage-1 A rows (v < 16), stage-2 X rows
    // (16 <= v < 32), then the X_P rows i0 .. i0 + 127 (v >= 32)
    auto unit_src = [&](int v, const uint16_t*& M, int& row0) {
      M = v < NUNIT ? At : Xt;
      row0 = v < NUNIT ? 32 * v : v < 2 * NUNIT ? 32 * (v - NUNIT) : i0 + 32 * (v - 2 * NUNIT);
    };
    // base: stream index of the stage's unit 0 (0 or 16); hf: the half
    auto khalf = [&](int base, int hf) {
      const bool xrows = base == NUNIT;
      // stage 2's unit 3 is loaded here rather than in stage 1's last unit,
      // so that the stage-1 epilogue (all accumulators live) holds three
      // units in flight, not four
      if (xrows && hf == 0) load_rows(Xt, 32 * (AHEAD - 1), ring[(NUNIT + AHEAD - 1) % NSLOT]);
      if (hf == 0) {
        write_rows(0, ring[base % NSLOT], xrows);
        write_rows(1, ring[base % NSLOT], xrows);
      }
      {
        const int ks0 = 2 * HUNIT * hf;
        const lds_u8* const rb = rfrag_base(ks0);
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) fb[ti] = *reinterpret_cast<const lds_u32x4*>(rb + 32768 * ti);
        read_fa(ks0, 0);
        read_fa(ks0, 1);
      }
#pragma unroll
      for (int uu = 0; uu < HUNIT; ++uu) {
        const int u = HUNIT * hf + uu;
        const uint16_t* M;
        int row0;
        unit_src(base + u + AHEAD, M, row0);
        Unit& dst = ring[(base + u + AHEAD) % NSLOT];
        const bool ld = xrows || u + AHEAD < NUNIT + AHEAD - 1;  // stage 2's unit 3: above
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int ks = 2 * u + s;
          const bool nx = ks + 1 < 2 * HUNIT * (hf + 1);  // k-step ks + 1 in this half
#pragma unroll
          for (int ti = 0; ti < 4; ++ti) acc[0][ti] = mfma(fa[0], fb[ti], acc[0][ti]);
          __builtin_amdgcn_sched_barrier(0);
          if (nx) read_fa(ks + 1, 0);
          if (ld) load_row(M, row0, dst, 2 * s);
          const lds_u8* const rb = nx ? rfrag_base(ks + 1) : lds;
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int ti = 0; ti < 4; ++ti) {
            acc[1][ti] = mfma(fa[1], fb[ti], acc[1][ti]);
            __builtin_amdgcn_sched_barrier(0);
            if (nx) fb[ti] = *reinterpret_cast<const lds_u32x4*>(rb + 32768 * ti);
            __builtin_amdgcn_sched_barrier(0);
          }
          if (nx) read_fa(ks + 1, 1);
          if (ks + 2 < NKS) write_rows(ks + 2, ring[(base + u + 1) % NSLOT], xrows);
          if (ld) load_row(M, row0, dst, 2 * s + 1);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };

    // ---- stage 1: c A_P A^T -----------------------------------------------------------
    // K loops at a raised wave priority: where one group's K loop meets the
    // other group's epilogue on a SIMD, the MFMA stream issues first
    __builtin_amdgcn_s_setprio(1);
    khalf(0, 0);
    lds_barrier();
    khalf(0, 1);
    __builtin_amdgcn_s_setprio(0);
    lds_barrier();

    // ---- stage-1 epilogue: B_P = bf16(c acc + b A_P) over A_P, own columns ----------
    // element (i = 32 ti + l32, j = col0 + 32 tj + 8 q + 4 hi + e): block
    // (4 ti + l32 / 8, col0 / 64), row l32 % 8, chunk 4 tj + q, bytes 8 hi ..
    {
      const int el = lane_o & 31, esw = r_swz(el);
      lds_u8* const ep1 = lds + 8192 * (el >> 3) + 1024 * (col0 >> 6) + 128 * (el & 7) + 8 * (lane_o >> 5);
      auto ep1_off = [&](int ti, int tj, int q) { return 32768 * ti + 16 * ((4 * tj + q) ^ esw); };
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        // all 8 A_P pieces of this row block first, one wait, then B_P over them
        u32x2_t av[2][4];
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            av[tj][q] = *reinterpret_cast<const lds_cu32x2*>(ep1 + ep1_off(ti, tj, q));
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
              y[e] = fmaf(cb, bf16_to_f32(half16(av[tj][q][e >> 1], e & 1)), cc * acc[tj][ti][4 * q + e]);
            *reinterpret_cast<lds_u32x2*>(ep1 + ep1_off(ti, tj, q)) =
                u32x2_t{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
          }
      }
    }
    lds_barrier();

#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

    // ---- stage 2: B_P X ---------------------------------------------------------------
    __builtin_amdgcn_s_setprio(1);
    khalf(NUNIT, 0);
    lds_barrier();
    khalf(NUNIT, 1);
    __builtin_amdgcn_s_setprio(0);
    lds_barrier();

    // ---- stage-2 epilogue -------------------------------------------------------------
    // X_P unit q (rows 32 q ..) sits in ring[(2 NUNIT + q) % NSLOT] = ring[q],
    // in the row layout of the stores (row 8 n + l / 8, columns 8 (l % 8) ..).
    const int el32 = lane_o & 31, ehi = lane_o >> 5, erow = lane_o >> 3, ech = lane_o & 7;
    UParam up;
    bool ufast = true;  // fused untile: blocks 2-3 both took the whole-vector path
    if constexpr (UDT >= 0) up = uparam_get(urec, usa);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      if (ti == 2 && more) {
        // The next item's A_P half grp into R (its last readers, the K2
        // halves of both groups over these block columns, are behind
        // barriers). Every X_P unit is waited for first (only blocks 0-1's
        // 8 stores and 8 ring loads may stay in flight), with the compiler's
        // own wait count, so that no wait for an X_P unit follows these
        // loads: it would also wait for them (vmcnt retires in order).
        wait_vm<16>();
        dma_half(nAt, ni0, grp, lane_o, cw_o);
      }
      const Unit& xp = ring[(2 * NUNIT + ti) % NSLOT];
      // the block's 32 result rows, in the row layout of the stores
      auto make_rows = [&](u32x4_t(&rows)[4]) {
        if constexpr (!ROUND_ONCE) {
          // bf16(B X) through W into the row layout, then + a X there with X_P
          // straight from the ring: the same operations on the same values as
          // in the accumulator layout, without staging X_P
#pragma unroll
          for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x16_t& v = acc[tj][ti];
              *reinterpret_cast<lds_u32x2*>(W + ep_off(el32, 4 * tj + q) + 8 * ehi) =
                  u32x2_t{pk_bf16(v[4 * q], v[4 * q + 1]), pk_bf16(v[4 * q + 2], v[4 * q + 3])};
            }
          // all 4 row reads, one wait
          u32x4_t bxr[4];
#pragma unroll
          for (int n = 0; n < 4; ++n) bxr[n] = *reinterpret_cast<const lds_u32x4*>(W + ep_off(8 * n + erow, ech));
#pragma unroll
          for (int n = 0; n < 4; ++n) {
            const u32x4_t x = SC ? scale8_rne(xp.v[n], xs) : xp.v[n];
#pragma unroll
            for (int w2 = 0; w2 < 4; ++w2) {
              const float y0 = fmaf(ca, __uint_as_float(x[w2] << 16), __uint_as_float(bxr[n][w2] << 16));
              const float y1 = fmaf(ca, __uint_as_float(x[w2] & 0xffff0000u), __uint_as_float(bxr[n][w2] & 0xffff0000u));
              rows[n][w2] = pk_bf16(y0, y1);
            }
          }
        } else {
          // bf16(B X + a X): X_P into the accumulator layout through W, the
          // fp32 sum there, the result back through W into rows
#pragma unroll
          for (int n = 0; n < 4; ++n)
            *reinterpret_cast<lds_u32x4*>(W + ep_off(8 * n + erow, ech)) = SC ? scale8_rne(xp.v[n], xs) : xp.v[n];
          // X_P in the accumulator layout: all 8 pieces, one wait
          u32x2_t xv[2][4];
#pragma unroll
          for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              xv[tj][q] = *reinterpret_cast<const lds_cu32x2*>(W + ep_off(el32, 4 * tj + q) + 8 * ehi);
#pragma unroll
          for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              float y[4];
#pragma unroll
              for (int e = 0; e < 4; ++e)
                y[e] = fmaf(ca, bf16_to_f32(half16(xv[tj][q][e >> 1], e & 1)), acc[tj][ti][4 * q + e]);
              *reinterpret_cast<lds_u32x2*>(W + ep_off(el32, 4 * tj + q) + 8 * ehi) =
                  u32x2_t{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
            }
          // the 32 result rows: all 4 row reads, one wait
#pragma unroll
          for (int n = 0; n < 4; ++n) rows[n] = *reinterpret_cast<const lds_u32x4*>(W + ep_off(8 * n + erow, ech));
        }
      };
      if constexpr (UDT >= 0) {
        // block 0's parameter loads after its staging: before it they would
        // be live beside all of the accumulators (and in the 2-D form, whose
        // staging holds more registers, every block's)
        bool f;
        if (ti == 0 || ROUND_ONCE)
          f = ba_untile_block<UDT, false>(up, g.u, make_rows, i0 + 32 * ti + erow, col0 + 8 * ech);
        else
          f = ba_untile_block<UDT, true>(up, g.u, make_rows, i0 + 32 * ti + erow, col0 + 8 * ech);
        if (ti >= 2) ufast = ufast && f;
      } else {
        u32x4_t rows[4];
        make_rows(rows);
#pragma unroll
        for (int n = 0; n < 4; ++n) gstore16(Yt + (i0 + 32 * ti + 8 * n) * T, xl_o, rows[n]);
      }
      // the next item's stage-1 unit ti into the slot X_P unit ti freed
      static_assert(AHEAD == 4, "one next-item unit per epilogue block");
      if (more) load_rows(nAt, 32 * ti, ring[ti]);
    }
    if (!more) break;
    // this group's half of the next A_P landed (issued before the
    // E2_VMEM_AFTER_DMA stores and loads above). With the fused untile, a
    // block on the element path may issue fewer than the 4 stores counted
    // (none at all outside the parameter): then only the ring loads are
    // certain to be younger than the direct-to-LDS loads.
    if (UDT < 0 || ufast)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(E2_VMEM_AFTER_DMA) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(E2_RING_AFTER_DMA) : "memory");
    lds_barrier();
    item = next;
  }
  // group 0 passes one extra barrier, meeting group 1's last segment
  if (grp == 0) lds_barrier();
}

int num_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

}  // namespace

bool ns5_ba_supported(int mp, int np) { return mp == T && np == T; }

bool ns5_ba_run(const uint16_t* A, const uint16_t* X, uint16_t* Y, const float* xinv, int64_t cnt, float a,
                float b, float c, bool round_once, hipStream_t s, const BaUntile* untile) {
  static_assert(kBaMaxTiles * (T / P) < (int64_t(1) << 31), "32-bit work-item indices");
  if (cnt < 1 || cnt > kBaMaxTiles) return false;
  const int64_t items = cnt * (T / P);
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t wgs_per_xcd = std::max<int64_t>(1, std::min<int64_t>(num_cus() / 8, per_xcd));
  const BaArgs args{A, X, Y, cnt, a, b, c, round_once ? 1 : 0, xinv, untile ? *untile : BaUntile{}};
  const dim3 grid((unsigned)(8 * wgs_per_xcd));
  if (untile) {
    if (xinv || !untile->params || untile->n_params <= 0 || !untile->sa || !untile->rec) return false;
    hipLaunchKernelGGL(untile_rec_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, s, *untile, cnt);
#define HM_BA_UNTILE(DT)                                                                      \
  if (round_once)                                                                            \
    hipLaunchKernelGGL((ns_ba_kernel<true, false, DT>), grid, dim3(NTH), 0, s, args);        \
  else                                                                                       \
    hipLaunchKernelGGL((ns_ba_kernel<false, false, DT>), grid, dim3(NTH), 0, s, args);
    switch (untile->param_dtype) {
      case HIMUON_DTYPE_F32: HM_BA_UNTILE(HIMUON_DTYPE_F32); break;
      case HIMUON_DTYPE_BF16: HM_BA_UNTILE(HIMUON_DTYPE_BF16); break;
      default: return false;  // fp16 parameters take the separate untile
    }
#undef HM_BA_UNTILE
    return true;
  }
  if (round_once && xinv)
    hipLaunchKernelGGL((ns_ba_kernel<true, true>), grid, dim3(NTH), 0, s, args);
  else if (round_once)
    hipLaunchKernelGGL((ns_ba_kernel<true, false>), grid, dim3(NTH), 0, s, args);
  else if (xinv)
    hipLaunchKernelGGL((ns_ba_kernel<false, true>), grid, dim3(NTH), 0, s, args);
  else
    hipLaunchKernelGGL((ns_ba_kernel<false, false>), grid, dim3(NTH), 0, s, args);
  return true;
}
