// The reference's three NS stage products for every operand dtype its kernels
// take: tl.dot on the loaded dtype with an fp32 accumulator, the result cast
// to the dtype of `out` (XXT.py:62-63, ba_plus_cAA.py:65-85,
// fused_bmm_add.py:73-88), tested there with bf16, fp16, fp32 and fp8 e5m2
// operands (tests/integration/test_kernels.py:36-165).
//
//   XXT          C = A A^T                     A: M x K       (mirrored store)
//   ba_plus_cAA  C = alpha A A^T + beta A      A: M x M       (mirrored store)
//   bmm_add      C = out(B X) + gamma X        B: M x M, X: M x N
//
// MFMA operands per input dtype (gfx950):
//   bf16          v_mfma_f32_32x32x16_bf16 on the values;
//   fp16          v_mfma_f32_32x32x16_f16 on the values;
//   fp8 e5m2      the same fp16 MFMA: an e5m2 byte is the upper byte of the
//                 fp16 with the same value (both have 5 exponent bits with
//                 bias 15), so widening is a shift and exact;
//   fp32          three bf16 MFMAs, hi*hi + hi*lo + lo*hi with hi = bf16(x)
//                 and lo = bf16(x - hi): 16 significant bits of every operand
//                 (TF32, which the reference's fp32 dot uses on its GPUs,
//                 keeps 11), each partial product exact in fp32.
// Output dtypes: fp32, bf16, fp16 (round to nearest even from fp32).
//
// The bf16-in / bf16-out products keep their own kernels (ns5.hip,
// ns5_stream.hip), bit-identical to torch; these kernels serve every other
// dtype pair. Block tile 128 x 128 x 64, four waves of 64 x 64 (2 x 2 MFMA
// 32x32 tiles), operands double-buffered in LDS, as ns5.hip's 128-block
// kernels; the Gram products compute the lower blocks and store each block
// and its mirror.
#include "ns5_kernels.h"

namespace {

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kLd = BK + 8;  // padded LDS row pitch (16-bit elements)

enum InType { kInF32 = HIMUON_DTYPE_F32, kInBf16 = HIMUON_DTYPE_BF16, kInF16 = HIMUON_DTYPE_F16,
              kInE5m2 = HIMUON_DTYPE_E5M2 };

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <int IN>
HM_DEV f32x16_t mfma_in(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (IN == kInF16 || IN == kInE5m2)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 8 consecutive input elements as 16-bit MFMA operands: `hi` always, `lo`
// (the fp32 remainder) for fp32 inputs.
struct Oct {
  u32x4_t hi, lo;
};

HM_DEV uint32_t e5m2_pair(uint32_t w, int k) {  // bytes 2k, 2k+1 of w -> two fp16
  const uint32_t b0 = (w >> (16 * k)) & 0xffu, b1 = (w >> (16 * k + 8)) & 0xffu;
  return (b0 << 8) | (b1 << 24);
}

template <int IN>
HM_DEV Oct load_oct(const void* base, int64_t idx) {
  Oct o;
  if constexpr (IN == kInF32) {
    const float* p = static_cast<const float*>(base) + idx;
    const f32x4_t v0 = *reinterpret_cast<const f32x4_t*>(p);
    const f32x4_t v1 = *reinterpret_cast<const f32x4_t*>(p + 4);
    float x[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float h0 = round_bf16(x[2 * k]), h1 = round_bf16(x[2 * k + 1]);
      o.hi[k] = pk_bf16(h0, h1);
      // (an infinite or NaN hi carries the value alone)
      o.lo[k] = pk_bf16(__builtin_isfinite(h0) ? x[2 * k] - h0 : 0.f, __builtin_isfinite(h1) ? x[2 * k + 1] - h1 : 0.f);
    }
  } else if constexpr (IN == kInE5m2) {
    const u32x2_t w = *reinterpret_cast<const u32x2_t*>(static_cast<const uint8_t*>(base) + idx);
    o.hi = u32x4_t{e5m2_pair(w[0], 0), e5m2_pair(w[0], 1), e5m2_pair(w[1], 0), e5m2_pair(w[1], 1)};
    o.lo = u32x4_t{0u, 0u, 0u, 0u};
  } else {
    o.hi = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(base) + idx);
    o.lo = u32x4_t{0u, 0u, 0u, 0u};
  }
  return o;
}

template <int IN>
HM_DEV float load_elem_in(const void* base, int64_t idx) {
  if constexpr (IN == kInF32) return static_cast<const float*>(base)[idx];
  else if constexpr (IN == kInBf16) return bf16_to_f32(static_cast<const uint16_t*>(base)[idx]);
  else if constexpr (IN == kInF16) return f16_to_f32(static_cast<const uint16_t*>(base)[idx]);
  else return f16_to_f32((uint16_t)(static_cast<const uint8_t*>(base)[idx] << 8));
}

HM_DEV float round_out(float v, int out_dtype) {
  if (out_dtype == HIMUON_DTYPE_BF16) return round_bf16(v);
  if (out_dtype == HIMUON_DTYPE_F16) return f16_to_f32(f32_to_f16(v));
  return v;
}

HM_DEV void store_out(void* base, int64_t idx, float v, int out_dtype) {
  if (out_dtype == HIMUON_DTYPE_F32)
    static_cast<float*>(base)[idx] = v;
  else if (out_dtype == HIMUON_DTYPE_BF16)
    static_cast<uint16_t*>(base)[idx] = (uint16_t)f32_to_bf16(v);
  else
    static_cast<uint16_t*>(base)[idx] = f32_to_f16(v);
}

constexpr int planes(int in) { return in == kInF32 ? 2 : 1; }

// C = alpha S S^T (+ beta S when add_s; K == M) for each batch entry; S:
// M x K, C: M x M. Lower 128 x 128 blocks only, each stored at (bi, bj) and
// mirrored.
template <int IN>
__global__ __launch_bounds__(kThreads) void prod_gram_kernel(const void* __restrict__ S, void* __restrict__ C,
                                                             int M, int K, int64_t ntiles, float alpha, float beta,
                                                             int add_s, int out_dtype) {
  constexpr int NP = planes(IN);
  __shared__ __attribute__((aligned(16))) uint16_t sI[2][NP][BM * kLd];
  __shared__ __attribute__((aligned(16))) uint16_t sJ[2][NP][BN * kLd];

  const int nb = M / BM;
  const int npairs = nb * (nb + 1) / 2;
  const int64_t total = ntiles * npairs;
  const int64_t item = xcd_item(total);
  if (item >= total) return;
  const int64_t tile = item / npairs;
  const int p = (int)(item % npairs);
  int bi = 0;
  while ((bi + 1) * (bi + 2) / 2 <= p) ++bi;
  const int bj = p - bi * (bi + 1) / 2;

  const int64_t s0 = tile * (int64_t)M * K;  // element index of the tile
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lrow = tid >> 3, lkv = (tid & 7) * 8;  // loader: rows lrow + 32q, k offset lkv

  Oct ra[4], rb[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = lrow + 32 * q;
      ra[q] = load_oct<IN>(S, s0 + (int64_t)(bi * BM + row) * K + k0 + lkv);
      rb[q] = load_oct<IN>(S, s0 + (int64_t)(bj * BN + row) * K + k0 + lkv);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = lrow + 32 * q;
      *reinterpret_cast<u32x4_t*>(&sI[buf][0][row * kLd + lkv]) = ra[q].hi;
      *reinterpret_cast<u32x4_t*>(&sJ[buf][0][row * kLd + lkv]) = rb[q].hi;
      if constexpr (NP == 2) {
        *reinterpret_cast<u32x4_t*>(&sI[buf][NP - 1][row * kLd + lkv]) = ra[q].lo;
        *reinterpret_cast<u32x4_t*>(&sJ[buf][NP - 1][row * kLd + lkv]) = rb[q].lo;
      }
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

  const int nk = K / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kk = ks * 16 + (lane >> 5) * 8;
      u32x4_t a[NP][2], b[NP][2];
#pragma unroll
      for (int pl = 0; pl < NP; ++pl)
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
          a[pl][mi] = *reinterpret_cast<const u32x4_t*>(&sI[cur][pl][(wm * 64 + mi * 32 + (lane & 31)) * kLd + kk]);
          b[pl][mi] = *reinterpret_cast<const u32x4_t*>(&sJ[cur][pl][(wn * 64 + mi * 32 + (lane & 31)) * kLd + kk]);
        }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          if constexpr (NP == 2) {
            acc[mi][ni] = mfma_in<IN>(a[1][mi], b[0][ni], acc[mi][ni]);
            acc[mi][ni] = mfma_in<IN>(a[0][mi], b[1][ni], acc[mi][ni]);
          }
          acc[mi][ni] = mfma_in<IN>(a[0][mi], b[0][ni], acc[mi][ni]);
        }
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // MFMA 32x32 output layout: register r of lane l holds row
  // 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
  const int64_t c0 = tile * (int64_t)M * M;
  const bool offdiag = bi > bj;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = bi * BM + wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int j = bj * BN + wn * 64 + ni * 32 + (lane & 31);
        float v = alpha * acc[mi][ni][r];
        if (add_s) v = fmaf(beta, load_elem_in<IN>(S, s0 + (int64_t)i * K + j), v);
        if (offdiag || i >= j) store_out(C, c0 + (int64_t)i * M + j, v, out_dtype);
        if (offdiag || i > j) store_out(C, c0 + (int64_t)j * M + i, v, out_dtype);
      }
}

// C = out(Bm X) + gamma X for each batch entry (Bm X rounded to the output
// dtype before the add: fused_bmm_add.py:73-88); Bm: M x M, X and C: M x N.
// X is the MFMA B operand with the contraction along its rows: each 4 x 8
// block of X is transposed into the k-octet-major LDS layout sX[k/8][j][k%8].
template <int IN>
__global__ __launch_bounds__(kThreads) void prod_apply_kernel(const void* __restrict__ Bm,
                                                              const void* __restrict__ X, void* __restrict__ C,
                                                              int M, int N, int64_t ntiles, float gamma,
                                                              int out_dtype) {
  constexpr int NP = planes(IN);
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][NP][BM * kLd];
  __shared__ __attribute__((aligned(16))) uint16_t sX[2][NP][(BK / 8) * BN * 8];

  const int nbi = M / BM, nbj = N / BN;
  const int blocks = nbi * nbj;
  const int64_t total = ntiles * blocks;
  const int64_t item = xcd_item(total);
  if (item >= total) return;
  const int64_t tile = item / blocks;
  const int blk = (int)(item % blocks);
  const int bi = blk / nbj, bj = blk % nbj;

  const int64_t b0 = tile * (int64_t)M * M, x0 = tile * (int64_t)M * N;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lrow = tid >> 3, lkv = (tid & 7) * 8;  // Bm loader
  const int xkq = tid >> 4, xjo = (tid & 15) * 8;  // X loader: rows 4 xkq .. + 3, columns xjo .. + 7

  Oct ra[4], rx[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = lrow + 32 * q;
      ra[q] = load_oct<IN>(Bm, b0 + (int64_t)(bi * BM + row) * M + k0 + lkv);
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) rx[rr] = load_oct<IN>(X, x0 + (int64_t)(k0 + 4 * xkq + rr) * N + bj * BN + xjo);
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = lrow + 32 * q;
      *reinterpret_cast<u32x4_t*>(&sA[buf][0][row * kLd + lkv]) = ra[q].hi;
      if constexpr (NP == 2) *reinterpret_cast<u32x4_t*>(&sA[buf][NP - 1][row * kLd + lkv]) = ra[q].lo;
    }
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
      uint16_t* base = &sX[buf][pl][(xkq >> 1) * BN * 8 + (xkq & 1) * 4];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e >> 1, h = e & 1;
        auto v = [&](int rr) { return pl == 0 ? rx[rr].hi[w] : rx[rr].lo[w]; };
        u32x2_t d;
        d[0] = pack2(half16(v(0), h), half16(v(1), h));
        d[1] = pack2(half16(v(2), h), half16(v(3), h));
        *reinterpret_cast<u32x2_t*>(base + (xjo + e) * 8) = d;
      }
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

  const int nk = M / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kk = ks * 16 + (lane >> 5) * 8;
      const int koct = ks * 2 + (lane >> 5);
      u32x4_t av[NP][2], bv[NP][2];
#pragma unroll
      for (int pl = 0; pl < NP; ++pl)
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
          av[pl][mi] = *reinterpret_cast<const u32x4_t*>(&sA[cur][pl][(wm * 64 + mi * 32 + (lane & 31)) * kLd + kk]);
          bv[pl][mi] = *reinterpret_cast<const u32x4_t*>(&sX[cur][pl][(koct * BN + wn * 64 + mi * 32 + (lane & 31)) * 8]);
        }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          if constexpr (NP == 2) {
            acc[mi][ni] = mfma_in<IN>(av[1][mi], bv[0][ni], acc[mi][ni]);
            acc[mi][ni] = mfma_in<IN>(av[0][mi], bv[1][ni], acc[mi][ni]);
          }
          acc[mi][ni] = mfma_in<IN>(av[0][mi], bv[0][ni], acc[mi][ni]);
        }
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = bi * BM + wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int j = bj * BN + wn * 64 + ni * 32 + (lane & 31);
        const int64_t e = x0 + (int64_t)i * N + j;
        const float bx = round_out(acc[mi][ni][r], out_dtype);
        store_out(C, e, bx + gamma * load_elem_in<IN>(X, e), out_dtype);
      }
}

bool dtype_in_ok(int d) {
  return d == HIMUON_DTYPE_F32 || d == HIMUON_DTYPE_BF16 || d == HIMUON_DTYPE_F16 || d == HIMUON_DTYPE_E5M2;
}
bool dtype_out_ok(int d) { return d == HIMUON_DTYPE_F32 || d == HIMUON_DTYPE_BF16 || d == HIMUON_DTYPE_F16; }

template <int IN>
void launch_gram(const void* s, void* c, int M, int K, int64_t items, int64_t batch, float alpha, float beta,
                 int add_s, int od, hipStream_t st) {
  hipLaunchKernelGGL(prod_gram_kernel<IN>, dim3((unsigned)xcd_grid(items)), dim3(kThreads), 0, st, s, c, M, K,
                     batch, alpha, beta, add_s, od);
}

template <int IN>
void launch_apply(const void* b, const void* x, void* c, int M, int N, int64_t items, int64_t batch, float gamma,
                  int od, hipStream_t st) {
  hipLaunchKernelGGL(prod_apply_kernel<IN>, dim3((unsigned)xcd_grid(items)), dim3(kThreads), 0, st, b, x, c, M, N,
                     batch, gamma, od);
}

// Work items (one 128 x 128 output block each) a launch takes: the grid is
// at most 2^31 workgroups.
constexpr int64_t kMaxItems = (int64_t(1) << 31) - 8;

int gram(const void* s, void* c, int M, int K, int64_t batch, float alpha, float beta, int add_s, int id, int od,
         void* stream) {
  if (!s || !c || s == c || batch < 0 || M <= 0 || K <= 0 || M % BM || K % BK || !dtype_in_ok(id) ||
      !dtype_out_ok(od) || (add_s && K != M))
    return HIMUON_EINVAL;
  if (batch == 0) return 0;
  const int nb = M / BM;
  if (batch > kMaxItems / (nb * (nb + 1) / 2)) return HIMUON_EINVAL;
  const int64_t items = batch * (nb * (nb + 1) / 2);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  switch (id) {
    case HIMUON_DTYPE_F32: launch_gram<kInF32>(s, c, M, K, items, batch, alpha, beta, add_s, od, st); break;
    case HIMUON_DTYPE_BF16: launch_gram<kInBf16>(s, c, M, K, items, batch, alpha, beta, add_s, od, st); break;
    case HIMUON_DTYPE_F16: launch_gram<kInF16>(s, c, M, K, items, batch, alpha, beta, add_s, od, st); break;
    default: launch_gram<kInE5m2>(s, c, M, K, items, batch, alpha, beta, add_s, od, st); break;
  }
  return (int)hipGetLastError();
}

}  // namespace

extern "C" int himuon_xxt_typed(const void* x, void* out, int64_t batch, int M, int K, int in_dtype,
                                int out_dtype, void* stream) {
  return gram(x, out, M, K, batch, 1.f, 0.f, 0, in_dtype, out_dtype, stream);
}

extern "C" int himuon_ba_plus_caa_typed(const void* a, void* out, int64_t batch, int M, float alpha, float beta,
                                        int in_dtype, int out_dtype, void* stream) {
  return gram(a, out, M, M, batch, alpha, beta, 1, in_dtype, out_dtype, stream);
}

extern "C" int himuon_bmm_add_typed(const void* b, const void* x, void* out, int64_t batch, int M, int N, float a,
                                    int in_dtype, int out_dtype, void* stream) {
  if (!b || !x || !out || out == x || out == b || batch < 0 || M <= 0 || N <= 0 || M % BM || N % BN ||
      !dtype_in_ok(in_dtype) || !dtype_out_ok(out_dtype))
    return HIMUON_EINVAL;
  if (batch == 0) return 0;
  const int64_t blocks = (int64_t)(M / BM) * (N / BN);
  if (batch > kMaxItems / blocks) return HIMUON_EINVAL;
  const int64_t items = batch * blocks;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  switch (in_dtype) {
    case HIMUON_DTYPE_F32: launch_apply<kInF32>(b, x, out, M, N, items, batch, a, out_dtype, st); break;
    case HIMUON_DTYPE_BF16: launch_apply<kInBf16>(b, x, out, M, N, items, batch, a, out_dtype, st); break;
    case HIMUON_DTYPE_F16: launch_apply<kInF16>(b, x, out, M, N, items, batch, a, out_dtype, st); break;
    default: launch_apply<kInE5m2>(b, x, out, M, N, items, batch, a, out_dtype, st); break;
  }
  return (int)hipGetLastError();
}
