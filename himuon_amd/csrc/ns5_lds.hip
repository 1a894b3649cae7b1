// Fused Newton-Schulz for NS tiles with mp == 128 (tile edges <= 128): one
// workgroup keeps a tile's X (128 x np) and its A / B (128 x 128) in LDS
// through all iterations, so HBM sees one read and one write of the tile.
// This is the LDS-resident counterpart of the reference's one-kernel NS5 for
// small tiles (triton_kernels/ns5_smem.py:46-104, dispatched for M*N <= 16384
// by himuon.py:263-284); the per-iteration rounding points are those of the
// three-kernel path (XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88):
//
//   X0 = bf16(x * inv)
//   A  = bf16(X X^T)                    lower 64x64 quadrants, mirrored
//   B  = bf16(c (A A^T) + b A)          lower 64x64 quadrants, mirrored
//   X' = bf16(bf16(B X) + a X)
//
// 256 threads = 4 waves. Gram products: the 10 lower 32x32 tiles (ti >= tj
// of the 4x4 grid of v_mfma_f32_32x32x16_bf16 tiles) are split 3, 3, 2, 2 over
// the four waves (GramPart), so every SIMD takes part; each strictly lower
// tile is also written mirrored. A diagonal tile is computed whole and is
// exactly symmetric (element (i, j) and (j, i) sum the same products in the
// same order). Apply: wave (wm, wn) computes rows 64 wm .. +63 and columns
// wn np/2 .. + np/2 - 1. Products accumulate in registers; the result
// replaces its LDS operand after a workgroup barrier. X is read as the MFMA
// B operand with the contraction along its rows through ds_read_b64_tr_b16.
// The next tile's X is loaded into registers while the current tile iterates.
// The k loops are unrolled fully, so the compiler issues later fragment reads
// ahead of the MFMAs that need them (7 % faster than 2- and 4-fold unrolling).
//
// LDS rows hold 16-byte chunks; chunk ch of row r sits at position
// ch ^ s(r), s(r) = 4 (r % 4) + (r / 4) % 4: 16 consecutive rows of one chunk
// (fragment reads) and 4 consecutive rows of 4 consecutive chunks
// (transposing reads, mirrored Gram stores) both cover all 16 bank groups.
// np = 128: 64 KiB per workgroup, two workgroups per CU; np = 256: 96 KiB.
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

// acc[k] = (S S^T) tile k of wave W, S = LDS operand with SCH chunks per row
// and K = 8 SCH columns. Lane holds element 4 q + e of acc[k] at
// C[32 ROW[I[k]] + l32][32 ROW[J[k]] + 8 q + 4 hi + e].
template <int W, int SCH>
HM_DEV void gram_mma(const lds_u8* S, int lane, f32x16_t (&acc)[3]) {
  using P = GramPart<W>;
  const int ln = opaque_lane(lane), l32 = ln & 31, hi = ln >> 5;
#pragma unroll
  for (int k = 0; k < P::NTL; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[k][e] = 0.f;
#pragma unroll
  for (int ks = 0; ks < SCH / 2; ++ks) {
    u32x4_t f[P::NR];
#pragma unroll
    for (int r = 0; r < P::NR; ++r)
      f[r] = *reinterpret_cast<lds_cu32x4*>(S + lds_pos(32 * P::ROW[r] + l32, 2 * ks + hi, SCH));
#pragma unroll
    for (int k = 0; k < P::NTL; ++k) acc[k] = mfma(f[P::J[k]], f[P::I[k]], acc[k]);
  }
}

// Store wave W's bf16 tiles o[k][q] (q: 4 columns each) into the 128 x 128
// LDS matrix C (ACH chunks per row), and the transpose of every strictly
// lower tile.
template <int W>
HM_DEV void gram_store(lds_u8* C, int lane, const u32x2_t (&o)[3][4]) {
  using P = GramPart<W>;
  constexpr int ACH = M / 8;
  const int ln = opaque_lane(lane), l32 = ln & 31, hi = ln >> 5;
#pragma unroll
  for (int k = 0; k < P::NTL; ++k) {
    const int ti = P::ROW[P::I[k]], tj = P::ROW[P::J[k]];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      *reinterpret_cast<lds_u32x2*>(C + lds_pos(32 * ti + l32, 4 * tj + q, ACH) + hi * 8) = o[k][q];
      if (ti != tj) {
        // after the quad transpose, lane (a = l32/4, kk = l32%4) holds
        // C^T[jt][it .. it + 3], jt = 32 tj + 8 q + 4 hi + kk, it = 32 ti + 4 a
        const int kk = ln & 3, a = l32 >> 2;
        const u32x2_t tv = quad_transpose(o[k][q], kk);
        const int jt = 32 * tj + 8 * q + 4 * hi + kk;
        *reinterpret_cast<lds_u32x2*>(C + lds_pos(jt, 4 * ti + (a >> 1), ACH) + (a & 1) * 8) = tv;
      }
    }
  }
}

// A = bf16(X X^T): wave W's tiles into A.
template <int W, int XCH>
HM_DEV void gram_a(const lds_u8* X, lds_u8* A, int lane) {
  f32x16_t acc[3];
  gram_mma<W, XCH>(X, lane, acc);
  u32x2_t o[3][4];
#pragma unroll
  for (int k = 0; k < GramPart<W>::NTL; ++k)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[k][q] = u32x2_t{pk_bf16(acc[k][4 * q], acc[k][4 * q + 1]), pk_bf16(acc[k][4 * q + 2], acc[k][4 * q + 3])};
  gram_store<W>(A, lane, o);
}

// B = bf16(c (A A^T) + b A) for wave W's tiles, into registers (A is still
// read by the other waves; the caller stores after a barrier).
template <int W>
HM_DEV void gram_b(const lds_u8* A, int lane, float cb, float cc, u32x2_t (&o)[3][4]) {
  using P = GramPart<W>;
  constexpr int ACH = M / 8;
  f32x16_t acc[3];
  gram_mma<W, ACH>(A, lane, acc);
  const int ln = opaque_lane(lane), l32 = ln & 31, hi = ln >> 5;
#pragma unroll
  for (int k = 0; k < P::NTL; ++k) {
    const int ti = P::ROW[P::I[k]], tj = P::ROW[P::J[k]];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x2_t rv = *reinterpret_cast<lds_cu32x2*>(A + lds_pos(32 * ti + l32, 4 * tj + q, ACH) + hi * 8);
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = fmaf(cb, bf16_to_f32(half16(rv[e >> 1], e & 1)), cc * acc[k][4 * q + e]);
      o[k][q] = u32x2_t{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
    }
  }
}

template <int NQ>
__global__ __launch_bounds__(NT, NQ == 1 ? 2 : 1) void ns5_lds_kernel(const uint16_t* x,
                                                        uint16_t* out,
                                                        const float* __restrict__ inv,
                                                        int64_t ntiles, int steps, float ca,
                                                        float cb, float cc, int round_once) {
  constexpr int N = 128 * NQ;   // NS columns (np)
  constexpr int XCH = N / 8;    // 16-byte chunks per X row
  constexpr int ACH = M / 8;    // chunks per A row
  __shared__ __attribute__((aligned(16))) uint8_t sx_raw[M * N * 2];
  __shared__ __attribute__((aligned(16))) uint8_t sa_raw[M * M * 2];
  lds_u8* const X = (lds_u8*)sx_raw;
  lds_u8* const A = (lds_u8*)sa_raw;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  // Transposing-read lane roles (Apply's X operand): lane (a', b') of each
  // 16-lane group addresses k-row 8 hi + a' (+ 4 for the second read) and
  // columns 16 ((lane >> 4) & 1) + 4 b' .. + 3 of a 32-column tile.
  const int r16 = lane & 15;
  const int tr_krow = 8 * hi + (r16 >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (r16 & 3);

  constexpr int VPT = M * XCH / NT;  // 16-byte chunks per thread
  u32x4_t v[VPT];                    // the tile to come, loaded ahead
  auto load_tile = [&](int64_t t) {
    const uint16_t* src = x + t * (int64_t)M * N;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = k * NT + tid;
      v[k] = *reinterpret_cast<const u32x4_t*>(src + (int64_t)(idx / XCH) * N + (idx % XCH) * 8);
    }
  };
  if (blockIdx.x < ntiles) load_tile(blockIdx.x);
  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    // ---- X0 = bf16(x * inv) into LDS ------------------------------------------
    const float sc = inv[t];
    __syncthreads();  // the previous tile's final LDS reads are done
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = k * NT + tid;
      *reinterpret_cast<lds_u32x4*>(X + lds_pos(idx / XCH, idx % XCH, XCH)) = scale8(v[k], sc);
    }
    // the next tile's loads run under this tile's iterations
    if (t + gridDim.x < ntiles) load_tile(t + gridDim.x);
    __syncthreads();

    for (int it = 0; it < steps; ++it) {
      // ---- A = bf16(X X^T) ------------------------------------------------------
      switch (wave) {
        case 0: gram_a<0, XCH>(X, A, lane); break;
        case 1: gram_a<1, XCH>(X, A, lane); break;
        case 2: gram_a<2, XCH>(X, A, lane); break;
        default: gram_a<3, XCH>(X, A, lane); break;
      }
      __syncthreads();

      // ---- B = bf16(c (A A^T) + b A), in place of A --------------------------------
      {
        u32x2_t o[3][4];
        switch (wave) {
          case 0: gram_b<0>(A, lane, cb, cc, o); break;
          case 1: gram_b<1>(A, lane, cb, cc, o); break;
          case 2: gram_b<2>(A, lane, cb, cc, o); break;
          default: gram_b<3>(A, lane, cb, cc, o); break;
        }
        __syncthreads();  // every read of A (products and the b A term) is done
        switch (wave) {
          case 0: gram_store<0>(A, lane, o); break;
          case 1: gram_store<1>(A, lane, o); break;
          case 2: gram_store<2>(A, lane, o); break;
          default: gram_store<3>(A, lane, o); break;
        }
      }
      __syncthreads();

      // ---- X' = bf16(bf16(B X) + a X), in place of X ------------------------------
      {
        constexpr int TJ = 2 * NQ;  // 32-column tiles per wave
        const int jb = wn * (N / 2);
        f32x16_t acc[TJ][2];
#pragma unroll
        for (int a = 0; a < TJ; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;
#pragma unroll
        for (int ks = 0; ks < M / 16; ++ks) {
          u32x4_t fb[2], fa[TJ];
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2)
            fb[t2] = *reinterpret_cast<lds_cu32x4*>(A + lds_pos(64 * wm + 32 * t2 + l32, 2 * ks + hi, ACH));
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj) {
            const int c0 = jb + 32 * tj + tr_col;
            const int kr = 16 * ks + tr_krow;
            const u32x2_t l2 = read_tr(X, lds_pos(kr, c0 >> 3, XCH) + (c0 & 7) * 2);
            const u32x2_t u2 = read_tr(X, lds_pos(kr + 4, c0 >> 3, XCH) + (c0 & 7) * 2);
            fa[tj] = u32x4_t{l2[0], l2[1], u2[0], u2[1]};
          }
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
        }
        u32x2_t o[2][TJ][4];
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int i = 64 * wm + 32 * ti + l32;
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
        __syncthreads();  // every read of X is done
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int i = 64 * wm + 32 * ti + l32;
              const int ch = (jb >> 3) + 4 * tj + q;
              *reinterpret_cast<lds_u32x2*>(X + lds_pos(i, ch, XCH) + hi * 8) = o[ti][tj][q];
            }
      }
      __syncthreads();
    }

    // ---- result -> global ----------------------------------------------------------
    uint16_t* dst = out + t * (int64_t)M * N;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = k * NT + tid;
      *reinterpret_cast<u32x4_t*>(dst + (int64_t)(idx / XCH) * N + (idx % XCH) * 8) =
          *reinterpret_cast<lds_cu32x4*>(X + lds_pos(idx / XCH, idx % XCH, XCH));
    }
  }
}

int num_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

}  // namespace

bool ns5_lds_supported(int mp, int np) { return mp == M && (np == 128 || np == 256); }

void ns5_lds_run(uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int mp, int np, int steps,
                 float a, float b, float c, bool round_once, hipStream_t s) {
  (void)mp;
  uint16_t* out = (steps & 1) ? y : x;
  const int64_t wgs = std::min<int64_t>(cnt, (int64_t)(np == 128 ? 2 : 1) * 4 * num_cus());
  if (np == 128)
    hipLaunchKernelGGL(ns5_lds_kernel<1>, dim3((unsigned)wgs), dim3(NT), 0, s, x, out, inv, cnt, steps, a, b, c, round_once ? 1 : 0);
  else
    hipLaunchKernelGGL(ns5_lds_kernel<2>, dim3((unsigned)wgs), dim3(NT), 0, s, x, out, inv, cnt, steps, a, b, c, round_once ? 1 : 0);
}
