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
// 256 threads = 4 waves. Gram products: waves (wm, wn) with wm >= wn compute
// their 64x64 quadrant (2x2 v_mfma_f32_32x32x16_bf16 tiles); wave (1, 0) also
// writes the mirror. Apply: wave (wm, wn) computes rows 64 wm .. +63 and
// columns wn np/2 .. + np/2 - 1. Products accumulate in registers; the result
// replaces its LDS operand after a workgroup barrier. X is read as the MFMA
// B operand with the contraction along its rows through ds_read_b64_tr_b16.
//
// LDS rows hold 16-byte chunks; chunk ch of row r sits at position
// ch ^ (r & 15), so 16 consecutive rows of one chunk cover all 64 banks.
// np = 128: 64 KiB per workgroup, two workgroups per CU; np = 256: 96 KiB.
#include "ns5_kernels.h"

namespace {

constexpr int NT = 256;
constexpr int M = 128;  // NS rows (mp)

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) u32x4_t lds_u32x4;

HM_DEV uint32_t lds_pos(int r, int ch, int chunks) {
  return (uint32_t)(r * chunks + (ch ^ (r & 15))) * 16u;
}

// Transposing read: 4 bf16 of the 8-byte row segment at `off`, redistributed
// across each group of 16 lanes (lane 4a + b receives element b of the
// segments addressed by lanes a, a + 4, a + 8, a + 12).
HM_DEV u32x2_t read_tr(const lds_u8* base, uint32_t off) {
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base + off));
  return __builtin_bit_cast(u32x2_t, r);
}

template <int NQ>
__global__ __launch_bounds__(NT, NQ == 1 ? 2 : 1) void ns5_lds_kernel(const uint16_t* __restrict__ x,
                                                        uint16_t* __restrict__ out,
                                                        const float* __restrict__ inv,
                                                        int64_t ntiles, int steps, float ca,
                                                        float cb, float cc) {
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
  const bool gram_wave = wm >= wn;
  const bool mirror_wave = wm > wn;
  // Transposing-read lane roles (Apply's X operand): lane (a', b') of each
  // 16-lane group addresses k-row 8 hi + a' (+ 4 for the second read) and
  // columns 16 ((lane >> 4) & 1) + 4 b' .. + 3 of a 32-column tile.
  const int r16 = lane & 15;
  const int tr_krow = 8 * hi + (r16 >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (r16 & 3);

  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    // ---- X0 = bf16(x * inv) into LDS ------------------------------------------
    constexpr int VPT = M * XCH / NT;  // 16-byte chunks per thread
    const uint16_t* src = x + t * (int64_t)M * N;
    const float sc = inv[t];
    u32x4_t v[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = k * NT + tid;
      v[k] = *reinterpret_cast<const u32x4_t*>(src + (int64_t)(idx / XCH) * N + (idx % XCH) * 8);
    }
    __syncthreads();  // the previous tile's final LDS reads are done
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = k * NT + tid;
      *reinterpret_cast<lds_u32x4*>(X + lds_pos(idx / XCH, idx % XCH, XCH)) = scale8(v[k], sc);
    }
    __syncthreads();

    for (int it = 0; it < steps; ++it) {
      // ---- A = bf16(X X^T) ------------------------------------------------------
      if (gram_wave) {
        f32x16_t acc[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;
#pragma unroll 4
        for (int ks = 0; ks < N / 16; ++ks) {
          u32x4_t fa[2], fb[2];
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2) {
            fb[t2] = *reinterpret_cast<lds_cu32x4*>(X + lds_pos(64 * wm + 32 * t2 + l32, 2 * ks + hi, XCH));
            fa[t2] = *reinterpret_cast<lds_cu32x4*>(X + lds_pos(64 * wn + 32 * t2 + l32, 2 * ks + hi, XCH));
          }
#pragma unroll
          for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int ti = 0; ti < 2; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
        }
        // lane holds A[i = 64 wm + 32 ti + l32][j = 64 wn + 32 tj + 8 q + 4 hi + e]
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
          for (int tj = 0; tj < 2; ++tj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x16_t& w = acc[tj][ti];
              const u32x2_t o = u32x2_t{pk_bf16(w[4 * q], w[4 * q + 1]), pk_bf16(w[4 * q + 2], w[4 * q + 3])};
              const int i = 64 * wm + 32 * ti + l32;
              *reinterpret_cast<lds_u32x2*>(A + lds_pos(i, 8 * wn + 4 * tj + q, ACH) + hi * 8) = o;
              if (mirror_wave) {
                // after the quad transpose, lane (a = l32/4, k = l32%4) holds
                // A^T[jt][it .. it + 3], jt = 64 wn + 32 tj + 8 q + 4 hi + k,
                // it = 64 wm + 32 ti + 4 a
                const int k = lane & 3, a = l32 >> 2;
                const u32x2_t tv = quad_transpose(o, k);
                const int jt = 64 * wn + 32 * tj + 8 * q + 4 * hi + k;
                *reinterpret_cast<lds_u32x2*>(A + lds_pos(jt, 8 * wm + 4 * ti + (a >> 1), ACH) + (a & 1) * 8) = tv;
              }
            }
      }
      __syncthreads();

      // ---- B = bf16(c (A A^T) + b A), in place of A --------------------------------
      {
        u32x2_t o[2][2][4];
        if (gram_wave) {
          f32x16_t acc[2][2];
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
              for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;
#pragma unroll 4
          for (int ks = 0; ks < M / 16; ++ks) {
            u32x4_t fa[2], fb[2];
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
              fb[t2] = *reinterpret_cast<lds_cu32x4*>(A + lds_pos(64 * wm + 32 * t2 + l32, 2 * ks + hi, ACH));
              fa[t2] = *reinterpret_cast<lds_cu32x4*>(A + lds_pos(64 * wn + 32 * t2 + l32, 2 * ks + hi, ACH));
            }
#pragma unroll
            for (int tj = 0; tj < 2; ++tj)
#pragma unroll
              for (int ti = 0; ti < 2; ++ti) acc[tj][ti] = mfma(fa[tj], fb[ti], acc[tj][ti]);
          }
#pragma unroll
          for (int ti = 0; ti < 2; ++ti)
#pragma unroll
            for (int tj = 0; tj < 2; ++tj)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int i = 64 * wm + 32 * ti + l32;
                const u32x2_t rv = *reinterpret_cast<lds_cu32x2*>(A + lds_pos(i, 8 * wn + 4 * tj + q, ACH) + hi * 8);
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  y[e] = fmaf(cb, bf16_to_f32(half16(rv[e >> 1], e & 1)), cc * acc[tj][ti][4 * q + e]);
                o[ti][tj][q] = u32x2_t{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
              }
        }
        __syncthreads();  // every read of A (products and the b A term) is done
        if (gram_wave) {
#pragma unroll
          for (int ti = 0; ti < 2; ++ti)
#pragma unroll
            for (int tj = 0; tj < 2; ++tj)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int i = 64 * wm + 32 * ti + l32;
                *reinterpret_cast<lds_u32x2*>(A + lds_pos(i, 8 * wn + 4 * tj + q, ACH) + hi * 8) = o[ti][tj][q];
                if (mirror_wave) {
                  const int k = lane & 3, a = l32 >> 2;
                  const u32x2_t tv = quad_transpose(o[ti][tj][q], k);
                  const int jt = 64 * wn + 32 * tj + 8 * q + 4 * hi + k;
                  *reinterpret_cast<lds_u32x2*>(A + lds_pos(jt, 8 * wm + 4 * ti + (a >> 1), ACH) + (a & 1) * 8) = tv;
                }
              }
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
#pragma unroll 2
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
                const float bx = bf16_to_f32(pk_bf16(acc[tj][ti][4 * q + e], 0.f) & 0xffffu);
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
                 float a, float b, float c, hipStream_t s) {
  (void)mp;
  uint16_t* out = (steps & 1) ? y : x;
  const int64_t wgs = std::min<int64_t>(cnt, (int64_t)(np == 128 ? 2 : 1) * 4 * num_cus());
  if (np == 128)
    hipLaunchKernelGGL(ns5_lds_kernel<1>, dim3((unsigned)wgs), dim3(NT), 0, s, x, out, inv, cnt, steps, a, b, c);
  else
    hipLaunchKernelGGL(ns5_lds_kernel<2>, dim3((unsigned)wgs), dim3(NT), 0, s, x, out, inv, cnt, steps, a, b, c);
}
