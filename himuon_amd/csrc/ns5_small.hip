// Newton-Schulz on NS tiles with few rows: m <= 64 rows (after the
// transpose-if-tall) of a tile whose buffer pads rows to mp = 128, run at
// their own height instead of the padded one. One workgroup keeps a tile's
// X (me x np, me = 16, 32 or 64, the first at least m) and its A and B
// (me x me) in LDS
// through all iterations; HBM sees the me rows read once and written once.
// This serves the shapes the reference routes to its fused small-tile kernel
// (M, N in {16 .. 1024}, M N <= 16384: himuon.py:261-284, ns5_smem.py:46-104)
// and its rectangular benchmark (exp_ns5_rect_bench.py:83-103), e.g. 16 x 1024,
// without paying for 128 rows. Rows me .. 127 of the buffer are never read
// or written: a zero row of X stays zero through NS, so the result's rows
// below m are those a 128-row computation gives.
//
// Per iteration, with the rounding points of the three-kernel path
// (XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88):
//   A  = bf16(X X^T)                   lower 16 x 16 tiles, v_mfma_f32_16x16x32_bf16
//   B  = bf16(c (A A^T) + b A)         lower 16 x 16 tiles, v_mfma_f32_16x16x16_bf16
//   X' = bf16(bf16(B X) + a X)         (bf16(B X + a X) with round_once)
// Each Gram tile is stored and mirrored, so A and B are exactly symmetric.
// Apply: wave w owns the 16-column blocks 2 w, 2 w + 1, 2 w + 8, 2 w + 9, ...
// (two per pass, B's fragments held in registers through the iteration); it
// keeps all me rows of its column blocks in registers until their k loop
// ends, then writes X' over its own columns of X (no other wave reads them).
// Workgroup barriers separate the products.
//
// MFMA 16x16 layouts: operand lane l holds row (A) or column (B) l % 16 and
// k = 8 (l / 16) .. + 7 (x32) or 4 (l / 16) .. + 3 (x16); result register r
// of lane l is element (4 (l / 16) + r, l % 16).
//
// LDS: X row-major, 16-byte chunk ch of row r at position ch ^ s(r),
// s(r) = 4 (r % 4) + (r / 4) % 4 (16 consecutive rows of one chunk, and 4
// rows of 2 consecutive chunks for the transposing reads, fall in distinct
// bank groups); A and B row-major with a pitch of me + 4 elements.
#include "ns5_kernels.h"

namespace {

constexpr int NT = 256;  // four waves
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) u32x4_t lds_u32x4;

HM_DEV f32x4_t mfma16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}
HM_DEV f32x4_t mfma16x16(u32x2_t a, u32x2_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4i16, a), __builtin_bit_cast(v4i16, b), c,
                                                   0, 0, 0);
}

HM_DEV uint32_t x_pos(int r, int ch, int chunks) {
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

HM_DEV uint16_t bf16_bits(float v) { return (uint16_t)(pk_bf16(v, 0.f) & 0xffffu); }

// ME: rows kept (multiple of 16, <= 64); NP: padded columns (multiple of 128).
template <int ME, int NP, bool ROUND_ONCE>
__global__ __launch_bounds__(NT) void ns5_small_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                       const float* __restrict__ inv, int64_t cnt, int steps,
                                                       float ca, float cb, float cc) {
  constexpr int T = ME / 16;          // 16-row blocks
  constexpr int CH = NP / 8;          // 16-byte chunks per X row
  constexpr int PA = ME + 4;          // A / B row pitch (elements)
  constexpr int X_BYTES = ME * NP * 2;
  constexpr int A_BYTES = ME * PA * 2;
  constexpr int NTILE = T * (T + 1) / 2;  // lower 16 x 16 tiles of A, B
  __shared__ __attribute__((aligned(16))) uint8_t lds_raw[X_BYTES + 2 * A_BYTES];
  lds_u8* const Xs = (lds_u8*)lds_raw;
  uint16_t* const As = reinterpret_cast<uint16_t*>(lds_raw + X_BYTES);
  uint16_t* const Bs = reinterpret_cast<uint16_t*>(lds_raw + X_BYTES + A_BYTES);
  auto lds16 = [&](uint16_t* base) { return (__attribute__((address_space(3))) uint16_t*)base; };

  const int64_t tile = blockIdx.x;
  if (tile >= cnt) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g4 = lane >> 4;
  const int64_t tile_elems = (int64_t)128 * NP;  // the buffer's padded tile

  // ---- X0 = bf16(x inv) of rows 0 .. ME - 1 into LDS -------------------------------------
  {
    const uint16_t* src = x + tile * tile_elems;
    const float s = inv[tile];
    for (int v = tid; v < ME * CH; v += NT) {
      const int r = v / CH, ch = v % CH;
      const u32x4_t q = *reinterpret_cast<const u32x4_t*>(src + (int64_t)r * NP + 8 * ch);
      *reinterpret_cast<lds_u32x4*>(Xs + x_pos(r, ch, CH)) = scale8_rne(q, s);
    }
  }
  __syncthreads();

  // lower tile p -> (ti, tj), ti >= tj
  auto tri = [](int p, int& ti, int& tj) {
    ti = 0;
    while ((ti + 1) * (ti + 2) / 2 <= p) ++ti;
    tj = p - ti * (ti + 1) / 2;
  };

  for (int it = 0; it < steps; ++it) {
    // ---- A = bf16(X X^T) ----------------------------------------------------------------
    for (int p = wave; p < NTILE; p += 4) {
      int ti, tj;
      tri(p, ti, tj);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int ks = 0; ks < NP / 32; ++ks) {
        const int ch = 4 * ks + g4;
        const u32x4_t a = *reinterpret_cast<const lds_u32x4*>(Xs + x_pos(16 * ti + l16, ch, CH));
        const u32x4_t b = *reinterpret_cast<const lds_u32x4*>(Xs + x_pos(16 * tj + l16, ch, CH));
        acc = mfma16x32(a, b, acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * ti + 4 * g4 + r, j = 16 * tj + l16;
        const uint16_t h = bf16_bits(acc[r]);
        lds16(As)[i * PA + j] = h;
        if (ti != tj) lds16(As)[j * PA + i] = h;  // (a diagonal tile is computed whole)
      }
    }
    __syncthreads();

    // ---- B = bf16(c (A A^T) + b A) ---------------------------------------------------------
    for (int p = wave; p < NTILE; p += 4) {
      int ti, tj;
      tri(p, ti, tj);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < T; ++ks) {
        const int k = 16 * ks + 4 * g4;
        const u32x2_t a = *reinterpret_cast<const __attribute__((address_space(3))) u32x2_t*>(
            lds16(As) + (16 * ti + l16) * PA + k);
        const u32x2_t b = *reinterpret_cast<const __attribute__((address_space(3))) u32x2_t*>(
            lds16(As) + (16 * tj + l16) * PA + k);
        acc = mfma16x16(a, b, acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * ti + 4 * g4 + r, j = 16 * tj + l16;
        const float v = fmaf(cb, bf16_to_f32(lds16(As)[i * PA + j]), cc * acc[r]);
        const uint16_t h = bf16_bits(v);
        lds16(Bs)[i * PA + j] = h;
        if (ti != tj) lds16(Bs)[j * PA + i] = h;
      }
    }
    __syncthreads();

    // ---- X' = bf16(bf16(B X) + a X), column blocks owned by the wave ------------------------
    // B's fragments are the same for every column block: read once per
    // iteration (T x T x 2 registers). Two column blocks per pass.
    u32x2_t bf[T][T];
#pragma unroll
    for (int ti = 0; ti < T; ++ti)
#pragma unroll
      for (int ks = 0; ks < T; ++ks)
        bf[ti][ks] = *reinterpret_cast<const __attribute__((address_space(3))) u32x2_t*>(
            lds16(Bs) + (16 * ti + l16) * PA + 16 * ks + 4 * g4);
    for (int cb0 = 2 * wave; cb0 < NP / 16; cb0 += 8) {
      f32x4_t acc[2][T];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ti = 0; ti < T; ++ti) acc[h][ti] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < T; ++ks) {
        // X[16 ks + 4 g4 .. + 3][16 cb + l16]: lane 4a + b of the group
        // addresses row 16 ks + 4 g4 + a', columns 16 cb + 4 b' .. + 3
        // (a' = l16 / 4, b' = l16 % 4)
        const int xr = 16 * ks + 4 * g4 + (l16 >> 2);
        u32x2_t xb[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int col = 16 * (cb0 + h) + 4 * (l16 & 3);
          xb[h] = read_tr(Xs, x_pos(xr, col >> 3, CH) + (col & 7) * 2);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int ti = 0; ti < T; ++ti) acc[h][ti] = mfma16x16(bf[ti][ks], xb[h], acc[h][ti]);
      }
      // every read of these columns is done (each lane waits for its own)
      // before any of them is overwritten: the reads above are this wave's
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ti = 0; ti < T; ++ti)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = 16 * ti + 4 * g4 + r, j = 16 * (cb0 + h) + l16;
            uint16_t* xe = reinterpret_cast<uint16_t*>(lds_raw + x_pos(i, j >> 3, CH) + (j & 7) * 2);
            const float xv = bf16_to_f32(*lds16(xe));
            const float bx = ROUND_ONCE ? acc[h][ti][r] : round_bf16(acc[h][ti][r]);
            *lds16(xe) = bf16_bits(fmaf(ca, xv, bx));
          }
    }
    __syncthreads();
  }

  // ---- result rows 0 .. ME - 1: x for an even step count, y for an odd one -------------------
  uint16_t* dst = ((steps & 1) ? y : const_cast<uint16_t*>(x)) + tile * tile_elems;
  for (int v = tid; v < ME * CH; v += NT) {
    const int r = v / CH, ch = v % CH;
    *reinterpret_cast<u32x4_t*>(dst + (int64_t)r * NP + 8 * ch) =
        *reinterpret_cast<const lds_u32x4*>(Xs + x_pos(r, ch, CH));
  }
}

template <int ME, int NP>
void launch(const uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int steps, float a, float b, float c,
            bool round_once, hipStream_t s) {
  if (round_once)
    hipLaunchKernelGGL((ns5_small_kernel<ME, NP, true>), dim3((unsigned)cnt), dim3(NT), 0, s, x, y, inv, cnt,
                       steps, a, b, c);
  else
    hipLaunchKernelGGL((ns5_small_kernel<ME, NP, false>), dim3((unsigned)cnt), dim3(NT), 0, s, x, y, inv, cnt,
                       steps, a, b, c);
}

template <int ME>
bool launch_np(int np, const uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int steps, float a, float b,
               float c, bool ro, hipStream_t s) {
  if (np == 128) { launch<ME, 128>(x, y, inv, cnt, steps, a, b, c, ro, s); return true; }
  if constexpr (ME <= 32) {
    switch (np) {
      case 256: launch<ME, 256>(x, y, inv, cnt, steps, a, b, c, ro, s); return true;
      case 384: launch<ME, 384>(x, y, inv, cnt, steps, a, b, c, ro, s); return true;
      case 512: launch<ME, 512>(x, y, inv, cnt, steps, a, b, c, ro, s); return true;
      case 768: launch<ME, 768>(x, y, inv, cnt, steps, a, b, c, ro, s); return true;
      case 1024: launch<ME, 1024>(x, y, inv, cnt, steps, a, b, c, ro, s); return true;
      default: break;
    }
  }
  if constexpr (ME <= 16) {
    if (np == 1536) { launch<ME, 1536>(x, y, inv, cnt, steps, a, b, c, ro, s); return true; }
    if (np == 2048) { launch<ME, 2048>(x, y, inv, cnt, steps, a, b, c, ro, s); return true; }
  }
  return false;
}

}  // namespace

int ns5_small_rows(int m) { return m <= 0 ? 0 : m <= 16 ? 16 : m <= 32 ? 32 : m <= 64 ? 64 : 0; }

// Admitted: me = 16 or 32 up to np = 2048 or 1024, me = 64 at np = 128 only:
// 64-row tiles with np >= 256 measured faster on the 128-row LDS-resident
// kernel (ns-rect sweep: 64 x 256 0.033 against 0.042 ms, 64 x 512 0.056
// against 0.061 ms; 64 x 128 0.030 against 0.030 ms).
bool ns5_small_supported(int m, int mp, int np) {
  const int me = ns5_small_rows(m);
  if (mp != 128 || me == 0) return false;
  if (me == 64) return np == 128;
  if (np == 128 || np == 256 || np == 384 || np == 512) return true;
  if (me <= 32 && (np == 768 || np == 1024)) return true;
  return me <= 16 && (np == 1536 || np == 2048);
}

bool ns5_small_run(const uint16_t* x, uint16_t* y, const float* inv, int64_t cnt, int m, int np, int steps,
                   float a, float b, float c, bool round_once, hipStream_t s) {
  if (cnt <= 0 || cnt > 0x7fffffff) return false;
  switch (ns5_small_rows(m)) {
    case 16: return launch_np<16>(np, x, y, inv, cnt, steps, a, b, c, round_once, s);
    case 32: return launch_np<32>(np, x, y, inv, cnt, steps, a, b, c, round_once, s);
    case 64: return launch_np<64>(np, x, y, inv, cnt, steps, a, b, c, round_once, s);
    default: return false;
  }
}
