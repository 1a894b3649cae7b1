// NS5 GEMM stages with 256x256 output blocks (NS tiles whose padded edges are
// multiples of 256: T = 256, 512, 1024 and the full-matrix shapes).
//
// 256 threads = 4 waves in a 2x2 grid; each wave owns a 128x128 sub-block as
// 4x4 tiles of v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per lane). The
// block's K slab (64) of both operands is double buffered in LDS (padded rows,
// 16-byte reads) with register prefetch of the slab after next.
//
// Operands are swapped relative to C = P Q: each MFMA computes a 32x32 tile of
// C^T, so lane l holds C[row l%32][4 consecutive columns] and the epilogue
// reads and writes 8-byte row segments directly.
//
//   gram:  C = bf16(alpha * S S^T + beta * S), lower blocks only; the block
//          (bi, bj), bi > bj, is also written mirrored at (bj, bi) through a
//          transposed LDS image. Diagonal blocks read one panel.
//   apply: Y = bf16(bf16(B X) + a X); X is contracted along its rows and is
//          staged k-octet-major (sX[k/8][j][k%8]) from 4x8 register blocks.
#include "ns5_kernels.h"

namespace {

constexpr int NT = 256;
constexpr int BT = 256;          // output block edge
constexpr int BK = 64;           // K slab
constexpr int LD = BK + 8;       // padded LDS row pitch of k-contiguous panels (elements)
constexpr int PANEL = BT * LD;   // elements per staged panel
constexpr int LDT = BT + 8;      // pitch of the transposed epilogue image

HM_DEV f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 256 rows x 64 k of a k-contiguous matrix: 2048 16-byte vectors, 8 per thread.
HM_DEV void gload_panel(u32x4_t (&r)[8], const uint16_t* __restrict__ base, int ld, int k0) {
  const int row = threadIdx.x >> 3, kv = (threadIdx.x & 7) * 8;
#pragma unroll
  for (int q = 0; q < 8; ++q)
    r[q] = *reinterpret_cast<const u32x4_t*>(base + (int64_t)(row + 32 * q) * ld + k0 + kv);
}

HM_DEV void lstore_panel(uint16_t* s, const u32x4_t (&r)[8], bool scaled, float sc) {
  const int row = threadIdx.x >> 3, kv = (threadIdx.x & 7) * 8;
#pragma unroll
  for (int q = 0; q < 8; ++q)
    *reinterpret_cast<u32x4_t*>(&s[(row + 32 * q) * LD + kv]) = scaled ? scale8(r[q], sc) : r[q];
}

// X[k0..k0+63][j0..j0+255] (row pitch ldx): two 4x8 blocks per thread.
HM_DEV void gload_xblock(u32x4_t (&r)[8], const uint16_t* __restrict__ X, int ldx, int k0, int j0) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int unit = threadIdx.x + NT * u;
    const int kq = unit >> 5, jo = (unit & 31) * 8;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      r[4 * u + rr] =
          *reinterpret_cast<const u32x4_t*>(X + (int64_t)(k0 + 4 * kq + rr) * ldx + j0 + jo);
  }
}

// Transpose the two 4x8 blocks into sX[k/8][j][k%8] (8-byte writes).
HM_DEV void lstore_xblock(uint16_t* sx, const u32x4_t (&r)[8], bool scaled, float sc) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int unit = threadIdx.x + NT * u;
    const int kq = unit >> 5, jo = (unit & 31) * 8;
    u32x4_t x[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) x[rr] = scaled ? scale8(r[4 * u + rr], sc) : r[4 * u + rr];
    uint16_t* base = sx + (kq >> 1) * BT * 8 + (kq & 1) * 4;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int w = e >> 1, h = e & 1;
      u32x2_t d;
      d[0] = pack2(half16(x[0][w], h), half16(x[1][w], h));
      d[1] = pack2(half16(x[2][w], h), half16(x[3][w], h));
      *reinterpret_cast<u32x2_t*>(base + (jo + e) * 8) = d;
    }
  }
}

HM_DEV void zero_acc(f32x16_t (&acc)[4][4]) {
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;
}

// ---------------------------------------------------------------------------
template <bool SCALED>
__global__ __launch_bounds__(NT, 1) void ns_gram256_kernel(
    const uint16_t* __restrict__ S, int64_t s_bs, int ldS, uint16_t* __restrict__ C, int64_t c_bs,
    int ldC, const float* __restrict__ inv, int M, int K, int64_t ntiles, float alpha,
    float beta) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[4 * PANEL];  // sI[2], sJ[2]
  const int nb = M / BT;
  const int npairs = nb * (nb + 1) / 2;
  const int64_t total = ntiles * npairs;
  const int64_t item = xcd_item(total);
  if (item >= total) return;
  const int64_t tile = item / npairs;
  const int p = (int)(item % npairs);
  int bi = 0;
  while ((bi + 1) * (bi + 2) / 2 <= p) ++bi;
  const int bj = p - bi * (bi + 1) / 2;
  const bool diag = bi == bj;

  const uint16_t* St = S + tile * s_bs;
  const uint16_t* Si = St + (int64_t)bi * BT * ldS;
  const uint16_t* Sj = St + (int64_t)bj * BT * ldS;
  constexpr bool scaled = SCALED;
  const float sc = scaled ? inv[tile] : 1.f;
  uint16_t* sI = smem;               // [2][PANEL]
  uint16_t* sJ = diag ? smem : smem + 2 * PANEL;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi = lane >> 5;

  u32x4_t ri[8], rj[8];
  f32x16_t acc[4][4];
  zero_acc(acc);

  const int nk = K / BK;
  gload_panel(ri, Si, ldS, 0);
  if (!diag) gload_panel(rj, Sj, ldS, 0);
  lstore_panel(sI, ri, scaled, sc);
  if (!diag) lstore_panel(sJ, rj, scaled, sc);
  if (nk > 1) {
    gload_panel(ri, Si, ldS, BK);
    if (!diag) gload_panel(rj, Sj, ldS, BK);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const uint16_t* cI = sI + (kt & 1) * PANEL;
    const uint16_t* cJ = sJ + (kt & 1) * PANEL;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kk = ks * 16 + hi * 8;
      u32x4_t fa[4], fb[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        // MFMA A operand = rows j (columns of C), B operand = rows i.
        fa[t] = *reinterpret_cast<const u32x4_t*>(&cJ[(wn * 128 + t * 32 + l32) * LD + kk]);
        fb[t] = *reinterpret_cast<const u32x4_t*>(&cI[(wm * 128 + t * 32 + l32) * LD + kk]);
      }
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
    }
    if (kt + 1 < nk) {
      lstore_panel(sI + ((kt + 1) & 1) * PANEL, ri, scaled, sc);
      if (!diag) lstore_panel(sJ + ((kt + 1) & 1) * PANEL, rj, scaled, sc);
      if (kt + 2 < nk) {
        gload_panel(ri, Si, ldS, (kt + 2) * BK);
        if (!diag) gload_panel(rj, Sj, ldS, (kt + 2) * BK);
      }
    }
    __syncthreads();
  }

  // Epilogue: lane holds C[i][j..j+3] for i = row0 + l32, j = col0 + 8q + 4hi.
  uint16_t* Ct = C + tile * c_bs;
  uint16_t* img = smem;  // transposed image [j][i], pitch LDT (off-diagonal blocks)
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
    const int il = wm * 128 + ti * 32 + l32;
    const int i = bi * BT + il;
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int jl = wn * 128 + tj * 32 + 8 * q + 4 * hi;
        const int j = bj * BT + jl;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = alpha * acc[tj][ti][4 * q + e];
        if (beta != 0.f) {
          const u32x2_t sv = *reinterpret_cast<const u32x2_t*>(St + (int64_t)i * ldS + j);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float s = bf16_to_f32(half16(sv[e >> 1], e & 1));
            if (scaled) s = round_bf16(s * sc);
            v[e] = fmaf(beta, s, v[e]);
          }
        }
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = f32_to_bf16(v[e]);
        u32x2_t o;
        o[0] = pack2(h[0], h[1]);
        o[1] = pack2(h[2], h[3]);
        *reinterpret_cast<u32x2_t*>(Ct + (int64_t)i * ldC + j) = o;
        if (!diag) {
#pragma unroll
          for (int e = 0; e < 4; ++e) img[(jl + e) * LDT + il] = (uint16_t)h[e];
        }
      }
    }
  }
  if (diag) return;
  __syncthreads();
  // Mirrored block (bj, bi): rows of the image are rows of C^T.
  for (int v = threadIdx.x; v < BT * (BT / 8); v += NT) {
    const int r = v >> 5, c8 = (v & 31) * 8;
    const u32x4_t q = *reinterpret_cast<const u32x4_t*>(&img[r * LDT + c8]);
    *reinterpret_cast<u32x4_t*>(Ct + (int64_t)(bj * BT + r) * ldC + bi * BT + c8) = q;
  }
}

// ---------------------------------------------------------------------------
template <bool SCALED>
__global__ __launch_bounds__(NT, 1) void ns_apply256_kernel(
    const uint16_t* __restrict__ Bm, int64_t b_bs, const uint16_t* __restrict__ X, int64_t x_bs,
    uint16_t* __restrict__ Y, int64_t y_bs, const float* __restrict__ inv, int M, int N,
    int64_t ntiles, float a) {
  __shared__ __attribute__((aligned(16))) uint16_t sB[2 * PANEL];
  __shared__ __attribute__((aligned(16))) uint16_t sX[2 * (BK / 8) * BT * 8];
  const int nbi = M / BT, nbj = N / BT;
  const int blocks = nbi * nbj;
  const int64_t total = ntiles * blocks;
  const int64_t item = xcd_item(total);
  if (item >= total) return;
  const int64_t tile = item / blocks;
  const int blk = (int)(item % blocks);
  const int bi = blk / nbj, bj = blk % nbj;

  const uint16_t* Bi = Bm + tile * b_bs + (int64_t)bi * BT * M;
  const uint16_t* Xt = X + tile * x_bs;
  constexpr bool scaled = SCALED;
  const float sc = scaled ? inv[tile] : 1.f;
  constexpr int XS = (BK / 8) * BT * 8;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi = lane >> 5;

  u32x4_t rb[8], rx[8];
  f32x16_t acc[4][4];
  zero_acc(acc);

  const int nk = M / BK;
  gload_panel(rb, Bi, M, 0);
  gload_xblock(rx, Xt, N, 0, bj * BT);
  lstore_panel(sB, rb, false, 1.f);
  lstore_xblock(sX, rx, scaled, sc);
  if (nk > 1) {
    gload_panel(rb, Bi, M, BK);
    gload_xblock(rx, Xt, N, BK, bj * BT);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const uint16_t* cB = sB + (kt & 1) * PANEL;
    const uint16_t* cX = sX + (kt & 1) * XS;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kk = ks * 16 + hi * 8;
      const int koct = ks * 2 + hi;
      u32x4_t fa[4], fb[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        // MFMA A operand = X columns j (k along X rows), B operand = Bm rows i.
        fa[t] = *reinterpret_cast<const u32x4_t*>(&cX[(koct * BT + wn * 128 + t * 32 + l32) * 8]);
        fb[t] = *reinterpret_cast<const u32x4_t*>(&cB[(wm * 128 + t * 32 + l32) * LD + kk]);
      }
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
    }
    if (kt + 1 < nk) {
      lstore_panel(sB + ((kt + 1) & 1) * PANEL, rb, false, 1.f);
      lstore_xblock(sX + ((kt + 1) & 1) * XS, rx, scaled, sc);
      if (kt + 2 < nk) {
        gload_panel(rb, Bi, M, (kt + 2) * BK);
        gload_xblock(rx, Xt, N, (kt + 2) * BK, bj * BT);
      }
    }
    __syncthreads();
  }

  uint16_t* Yt = Y + tile * y_bs;
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
    const int i = bi * BT + wm * 128 + ti * 32 + l32;
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = bj * BT + wn * 128 + tj * 32 + 8 * q + 4 * hi;
        const u32x2_t xv = *reinterpret_cast<const u32x2_t*>(Xt + (int64_t)i * N + j);
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = bf16_to_f32(half16(xv[e >> 1], e & 1));
          if (scaled) x = round_bf16(x * sc);
          const float bx = round_bf16(acc[tj][ti][4 * q + e]);
          h[e] = f32_to_bf16(fmaf(a, x, bx));
        }
        u32x2_t o;
        o[0] = pack2(h[0], h[1]);
        o[1] = pack2(h[2], h[3]);
        *reinterpret_cast<u32x2_t*>(Yt + (int64_t)i * N + j) = o;
      }
    }
  }
}

}  // namespace

void ns5_launch_gram256(const uint16_t* S, int64_t s_bs, int ldS, uint16_t* C, int64_t c_bs,
                        int ldC, const float* inv, int M, int K, int64_t ntiles, float alpha,
                        float beta, hipStream_t s) {
  const int nb = M / BT;
  const int64_t items = ntiles * (nb * (nb + 1) / 2);
  if (inv)
    hipLaunchKernelGGL(ns_gram256_kernel<true>, dim3((unsigned)xcd_grid(items)), dim3(NT), 0, s, S,
                       s_bs, ldS, C, c_bs, ldC, inv, M, K, ntiles, alpha, beta);
  else
    hipLaunchKernelGGL(ns_gram256_kernel<false>, dim3((unsigned)xcd_grid(items)), dim3(NT), 0, s, S,
                       s_bs, ldS, C, c_bs, ldC, inv, M, K, ntiles, alpha, beta);
}

void ns5_launch_apply256(const uint16_t* Bm, int64_t b_bs, const uint16_t* X, int64_t x_bs,
                         uint16_t* Y, int64_t y_bs, const float* inv, int M, int N, int64_t ntiles,
                         float a, hipStream_t s) {
  const int64_t items = ntiles * (M / BT) * (N / BT);
  if (inv)
    hipLaunchKernelGGL(ns_apply256_kernel<true>, dim3((unsigned)xcd_grid(items)), dim3(NT), 0, s,
                       Bm, b_bs, X, x_bs, Y, y_bs, inv, M, N, ntiles, a);
  else
    hipLaunchKernelGGL(ns_apply256_kernel<false>, dim3((unsigned)xcd_grid(items)), dim3(NT), 0, s,
                       Bm, b_bs, X, x_bs, Y, y_bs, inv, M, N, ntiles, a);
}
