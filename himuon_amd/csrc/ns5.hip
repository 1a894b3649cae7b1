// Batched quintic Newton-Schulz (NS5) on gfx950 bf16 MFMA, fp32 accumulation.
//
// Per NS tile (m x n, m <= n, zero padded to mp x np) and per iteration:
//   A = bf16(X X^T)                      -> ns_gram_kernel (alpha=1, beta=0)
//   B = bf16(c A A^T + b A)              -> ns_gram_kernel (alpha=c, beta=b)
//   X = bf16(bf16(B X) + a X)            -> ns_apply_kernel
// following the rounding points of the reference kernels
// (triton_kernels/XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88,
// ns5_smem.py:84-101). A and B are symmetric: the gram kernel computes only
// the lower-triangular 128x128 blocks and stores each block twice (as itself
// and mirrored), so both products cost half the dense FLOPs.
//
// Iteration 0 reads the raw bf16 tile and applies the per-tile Frobenius
// normaliser while staging operands into LDS: X0 = bf16(x * inv[t])
// (himuon.py:242, ns5_smem.py:84-87).
//
// Block tile 128x128x64, 256 threads = 4 waves in a 2x2 grid, each wave owns a
// 64x64 sub-block = 2x2 MFMA 32x32x16 tiles. Operands are double buffered in
// LDS with register prefetch of the next K slab. Blocks are mapped to XCDs so
// all blocks of one NS tile share an L2.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "ns5_kernels.h"

namespace {

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kLd = BK + 8;  // padded LDS row pitch (elements) of k-contiguous operands

HM_DEV f32x16_t mfma_32x32x16(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// C = bf16(alpha * S S^T + beta * S) for each tile; S is M x K (row pitch ldS),
// C is M x M (row pitch ldC). Only blocks bi >= bj are computed; every block
// is written at (bi, bj) and mirrored at (bj, bi), so C is exactly symmetric.
// beta != 0 requires K == M (S square).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads, 2) void ns_gram_kernel(
    const uint16_t* __restrict__ S, int64_t s_bs, int ldS, uint16_t* __restrict__ C,
    int64_t c_bs, int ldC, const float* __restrict__ inv, int M, int K, int64_t ntiles,
    float alpha, float beta) {
  __shared__ __attribute__((aligned(16))) uint16_t sI[2][BM * kLd];
  __shared__ __attribute__((aligned(16))) uint16_t sJ[2][BN * kLd];

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

  const uint16_t* St = S + tile * s_bs;
  const uint16_t* Si = St + (int64_t)bi * BM * ldS;
  const uint16_t* Sj = St + (int64_t)bj * BN * ldS;
  const bool scaled = inv != nullptr;
  const float sc = scaled ? inv[tile] : 1.f;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lrow = tid >> 3, lkv = (tid & 7) * 8;  // loader: rows lrow + 32q, k offset lkv

  u32x4_t ra[4], rb[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = lrow + 32 * q;
      ra[q] = *reinterpret_cast<const u32x4_t*>(Si + (int64_t)row * ldS + k0 + lkv);
      rb[q] = *reinterpret_cast<const u32x4_t*>(Sj + (int64_t)row * ldS + k0 + lkv);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = lrow + 32 * q;
      u32x4_t a = ra[q], b = rb[q];
      if (scaled) {
        a = scale8(a, sc);
        b = scale8(b, sc);
      }
      *reinterpret_cast<u32x4_t*>(&sI[buf][row * kLd + lkv]) = a;
      *reinterpret_cast<u32x4_t*>(&sJ[buf][row * kLd + lkv]) = b;
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
      u32x4_t a[2], b[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
        a[mi] = *reinterpret_cast<const u32x4_t*>(
            &sI[cur][(wm * 64 + mi * 32 + (lane & 31)) * kLd + kk]);
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
        b[ni] = *reinterpret_cast<const u32x4_t*>(
            &sJ[cur][(wn * 64 + ni * 32 + (lane & 31)) * kLd + kk]);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma_32x32x16(a[mi], b[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue. MFMA 32x32 output layout: register r of lane l holds
  // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  uint16_t* Ct = C + tile * c_bs;
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
        if (beta != 0.f) {
          float s = bf16_to_f32(St[(int64_t)i * ldS + j]);
          if (scaled) s = round_bf16(s * sc);
          v = fmaf(beta, s, v);
        }
        const uint16_t h = (uint16_t)f32_to_bf16(v);
        if (offdiag || i >= j) Ct[(int64_t)i * ldC + j] = h;
        if (offdiag || i > j) Ct[(int64_t)j * ldC + i] = h;
      }
}

// ---------------------------------------------------------------------------
// Y = bf16(bf16(Bm X) + a X) for each tile; Bm is M x M symmetric (pitch M),
// X and Y are M x N (pitch N). X is the MFMA B operand with the contraction
// along its rows, so each 4x8 register block of X is transposed into a
// k-octet-major LDS layout sX[k/8][j][k%8] that serves 16-byte operand reads.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads, 2) void ns_apply_kernel(
    const uint16_t* __restrict__ Bm, int64_t b_bs, const uint16_t* __restrict__ X, int64_t x_bs,
    uint16_t* __restrict__ Y, int64_t y_bs, const float* __restrict__ inv, int M, int N,
    int64_t ntiles, float a, int round_once) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * kLd];
  __shared__ __attribute__((aligned(16))) uint16_t sX[2][(BK / 8) * BN * 8];

  const int nbi = M / BM, nbj = N / BN;
  const int blocks = nbi * nbj;
  const int64_t total = ntiles * blocks;
  const int64_t item = xcd_item(total);
  if (item >= total) return;
  const int64_t tile = item / blocks;
  const int blk = (int)(item % blocks);
  const int bi = blk / nbj, bj = blk % nbj;

  const uint16_t* Ai = Bm + tile * b_bs + (int64_t)bi * BM * M;
  const uint16_t* Xt = X + tile * x_bs;
  const bool scaled = inv != nullptr;
  const float sc = scaled ? inv[tile] : 1.f;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lrow = tid >> 3, lkv = (tid & 7) * 8;    // Bm loader
  const int xkq = tid >> 4, xjo = (tid & 15) * 8;    // X loader: rows 4*xkq..+3, cols xjo..+7

  u32x4_t ra[4], rx[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = lrow + 32 * q;
      ra[q] = *reinterpret_cast<const u32x4_t*>(Ai + (int64_t)row * M + k0 + lkv);
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      rx[rr] = *reinterpret_cast<const u32x4_t*>(Xt + (int64_t)(k0 + 4 * xkq + rr) * N +
                                                 bj * BN + xjo);
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = lrow + 32 * q;
      *reinterpret_cast<u32x4_t*>(&sA[buf][row * kLd + lkv]) = ra[q];
    }
    u32x4_t x[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) x[rr] = scaled ? scale8(rx[rr], sc) : rx[rr];
    uint16_t* base = &sX[buf][(xkq >> 1) * BN * 8 + (xkq & 1) * 4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int w = e >> 1, h = e & 1;
      u32x2_t d;
      d[0] = pack2(half16(x[0][w], h), half16(x[1][w], h));
      d[1] = pack2(half16(x[2][w], h), half16(x[3][w], h));
      *reinterpret_cast<u32x2_t*>(base + (xjo + e) * 8) = d;
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
      u32x4_t av[2], bv[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
        av[mi] = *reinterpret_cast<const u32x4_t*>(
            &sA[cur][(wm * 64 + mi * 32 + (lane & 31)) * kLd + kk]);
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
        bv[ni] = *reinterpret_cast<const u32x4_t*>(
            &sX[cur][(koct * BN + wn * 64 + ni * 32 + (lane & 31)) * 8]);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma_32x32x16(av[mi], bv[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  uint16_t* Yt = Y + tile * y_bs;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = bi * BM + wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int j = bj * BN + wn * 64 + ni * 32 + (lane & 31);
        float xv = bf16_to_f32(Xt[(int64_t)i * N + j]);
        if (scaled) xv = round_bf16(xv * sc);
        const float bx = round_once ? acc[mi][ni][r] : round_bf16(acc[mi][ni][r]);
        Yt[(int64_t)i * N + j] = (uint16_t)f32_to_bf16(fmaf(a, xv, bx));
      }
}

// Y = bf16(X * inv[t]) (steps == 0) or a plain copy (inv == nullptr).
__global__ __launch_bounds__(kThreads) void ns_scale_copy_kernel(const uint16_t* __restrict__ X,
                                                                uint16_t* __restrict__ Y,
                                                                const float* __restrict__ inv,
                                                                int64_t per_tile, int64_t ntiles) {
  const int64_t nvec = ntiles * per_tile / 8;
  for (int64_t v = (int64_t)blockIdx.x * kThreads + threadIdx.x; v < nvec;
       v += (int64_t)gridDim.x * kThreads) {
    u32x4_t q = reinterpret_cast<const u32x4_t*>(X)[v];
    if (inv) q = scale8(q, inv[(v * 8) / per_tile]);
    reinterpret_cast<u32x4_t*>(Y)[v] = q;
  }
}

}  // namespace

extern "C" size_t himuon_ns5_workspace_bytes(int64_t sub_batch, int mp, int np) {
  if (sub_batch <= 0 || mp <= 0 || np <= 0) return 0;
  return 2 * (size_t)sub_batch * mp * mp * sizeof(uint16_t);  // A and B per sub-batch tile
}

namespace {
// himuon_ns5_ex, and with `untile` (himuon_ns5_untile_apply; the caller has
// checked that the fused path applies) the untile with WD/LR fused into the
// last iteration: its tile0 is the bucket index of tile 0 of x.
int ns5_impl(uint16_t* x, uint16_t* y, const float* inv, int64_t n_tiles, int mp, int np, int steps, float a,
             float b, float c, void* workspace, size_t workspace_bytes, int64_t sub_batch, int flags,
             void* stream, const BaUntile* untile) {
  const int family = flags & HIMUON_NS_FAMILY_MASK;
  const bool round_once = (flags & HIMUON_NS_ROUND_ONCE) != 0;
  const int rows = (flags & HIMUON_NS_ROWS_MASK) >> HIMUON_NS_ROWS_SHIFT;
  if (!x || !y || x == y || !inv || n_tiles < 0 || steps < 0 || mp <= 0 || np <= 0 || mp > np ||
      mp % HIMUON_NS_ALIGN || np % HIMUON_NS_ALIGN || sub_batch <= 0 || rows > 64 ||
      (flags & ~(HIMUON_NS_FAMILY_MASK | HIMUON_NS_ROUND_ONCE | HIMUON_NS_ROWS_MASK)) ||
      (family != HIMUON_NS_FAMILY_AUTO && family != HIMUON_NS_FAMILY_BLOCK128 &&
       family != HIMUON_NS_FAMILY_STREAM3))
    return HIMUON_EINVAL;
  if (n_tiles == 0) return 0;
  const int64_t sb = sub_batch < n_tiles ? sub_batch : n_tiles;
  if (steps > 0 && (!workspace || workspace_bytes < himuon_ns5_workspace_bytes(sb, mp, np)))
    return HIMUON_ENOSPC;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t sq = (int64_t)mp * mp, rect = (int64_t)mp * np;

  if (steps == 0) {  // X0 = bf16(x * inv), in place (the result of an even step count is in x)
    const int64_t nvec = n_tiles * rect / 8;
    const unsigned grid = (unsigned)std::min<int64_t>((nvec + kThreads - 1) / kThreads, 65536);
    hipLaunchKernelGGL(ns_scale_copy_kernel, dim3(grid), dim3(kThreads), 0, s, x, x, inv, rect,
                       n_tiles);
    return (int)hipGetLastError();
  }

  uint16_t* wsA = static_cast<uint16_t*>(workspace);
  uint16_t* wsB = wsA + sb * sq;
  // Family AUTO: tiles whose padded edges are multiples of 256 run the
  // persistent streamed-operand kernels (ns5_stream.hip); tiles with mp == 128
  // and np in {128, 256, 512} run the fused LDS-resident kernel (ns5_lds.hip); other tiles
  // run the 128-block kernels below, which family BLOCK128 selects for every
  // geometry.
  // 512 x 512 tiles run the first product on the stream kernels and the
  // other two fused (ns5_ba.hip); family STREAM3 keeps three stream kernels.
  const bool small = family == HIMUON_NS_FAMILY_BLOCK128;
  const bool few_rows = family == HIMUON_NS_FAMILY_AUTO && ns5_small_supported(rows, mp, np);
  const bool st = ns5_stream_supported(mp, np) && !small;
  const bool lds = ns5_lds_supported(mp, np) && !small;
  const bool ba = ns5_ba_supported(mp, np) && family == HIMUON_NS_FAMILY_AUTO;
  const int nb = mp / BM;
  const int npairs = nb * (nb + 1) / 2;
  const int apply_blocks = (mp / BM) * (np / BN);

  for (int64_t s0 = 0; s0 < n_tiles; s0 += sb) {
    const int64_t cnt = std::min<int64_t>(sb, n_tiles - s0);
    const int64_t o = s0 * rect;
    if (few_rows) {
      if (!ns5_small_run(x + o, y + o, inv + s0, cnt, rows, np, steps, a, b, c, round_once, s)) return HIMUON_EINVAL;
    } else if (lds) {
      ns5_lds_run(x + o, y + o, inv + s0, cnt, mp, np, steps, a, b, c, round_once, s);
    } else if (st) {
      BaUntile u{};
      if (untile) {
        u = *untile;
        u.tile0 += s0;
      }
      const int rc = ns5_stream_run(x + o, y + o, inv + s0, cnt, mp, np, steps, a, b, c, round_once, ba, wsA,
                                    wsB, s, untile ? &u : nullptr);
      if (rc) return rc;
    } else {
      const uint16_t* cur = x + o;
      uint16_t* nxt = y + o;
      const float* cur_inv = inv + s0;
      for (int it = 0; it < steps; ++it) {
        hipLaunchKernelGGL(ns_gram_kernel, dim3((unsigned)xcd_grid(cnt * npairs)),
                           dim3(kThreads), 0, s, cur, rect, np, wsA, sq, mp, cur_inv, mp, np,
                           cnt, 1.0f, 0.0f);
        hipLaunchKernelGGL(ns_gram_kernel, dim3((unsigned)xcd_grid(cnt * npairs)),
                           dim3(kThreads), 0, s, wsA, sq, mp, wsB, sq, mp, nullptr, mp, mp, cnt,
                           c, b);
        hipLaunchKernelGGL(ns_apply_kernel, dim3((unsigned)xcd_grid(cnt * apply_blocks)),
                           dim3(kThreads), 0, s, wsB, sq, cur, rect, nxt, rect, cur_inv, mp, np,
                           cnt, a, round_once ? 1 : 0);
        const uint16_t* t = cur;
        cur = nxt;
        nxt = const_cast<uint16_t*>(t);
        cur_inv = nullptr;
      }
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  return 0;
}
}  // namespace

extern "C" int himuon_ns5_ex(uint16_t* x, uint16_t* y, const float* inv, int64_t n_tiles, int mp,
                             int np, int steps, float a, float b, float c, void* workspace,
                             size_t workspace_bytes, int64_t sub_batch, int flags, void* stream) {
  return ns5_impl(x, y, inv, n_tiles, mp, np, steps, a, b, c, workspace, workspace_bytes, sub_batch, flags, stream,
                  nullptr);
}

extern "C" int himuon_ns5_untile_apply_supported(int mp, int np, int tile_h, int tile_w, int steps, int flags,
                                                 int param_dtype) {
  const int family = flags & HIMUON_NS_FAMILY_MASK;
  return ns5_ba_supported(mp, np) && family == HIMUON_NS_FAMILY_AUTO && steps >= 2 && tile_h >= 1 &&
         tile_h <= tile_w && tile_w <= np && tile_h <= mp &&
         (param_dtype == HIMUON_DTYPE_F32 || param_dtype == HIMUON_DTYPE_BF16);
}

extern "C" int himuon_ns5_untile_apply(uint16_t* x, uint16_t* y, const float* inv, int64_t n_tiles, int mp, int np,
                                       int steps, float a, float b, float c, void* workspace,
                                       size_t workspace_bytes, int64_t sub_batch, int flags,
                                       const HimuonParamDesc* params_dev, int n_params, int64_t tile_begin,
                                       int tile_h, int tile_w, int param_dtype, const float* scale_alpha_dev,
                                       void* stream) {
  if (!himuon_ns5_untile_apply_supported(mp, np, tile_h, tile_w, steps, flags, param_dtype) || !params_dev ||
      n_params <= 0 || tile_begin < 0 || !scale_alpha_dev)
    return HIMUON_EINVAL;
  const BaUntile u{params_dev, n_params, tile_begin, tile_h, tile_w, param_dtype, scale_alpha_dev};
  return ns5_impl(x, y, inv, n_tiles, mp, np, steps, a, b, c, workspace, workspace_bytes, sub_batch, flags, stream,
                  &u);
}

// ---------------------------------------------------------------------------
// Allocation-free NS5: the A/B workspace is a file-scope device array (one
// copy per GPU, held until the process ends). Its device address is looked
// up once per device with that device current; host code uses only that
// address, never the array's name (a host-side stand-in).
// ---------------------------------------------------------------------------
namespace {
__device__ __align__(256) uint8_t scratch[HIMUON_NS_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_dev[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of this device's `scratch`, or nullptr (err set).
void* scratch_address(int* err) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = (int)e;
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *err = HIMUON_EINVAL;
    return nullptr;
  }
  void* p = g_scratch_dev[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_dev[dev].load(std::memory_order_relaxed);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *err = e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
      return nullptr;
    }
    g_scratch_dev[dev].store(p, std::memory_order_release);
  }
  return p;
}
}  // namespace

extern "C" int himuon_lds_step(const HimuonParamDesc* params_dev, int n_params, int64_t tile_begin,
                               int64_t n_tiles, int tile_h, int tile_w, int dtype, int param_dtype, int steps,
                               float a, float b, float c, float eps, int flags, const float* scale_alpha_dev,
                               void* stream) {
  if (!params_dev || n_params <= 0 || tile_begin < 0 || n_tiles < 0 || steps < 0 || !scale_alpha_dev ||
      (flags & ~HIMUON_NS_ROUND_ONCE) || !lds_step_supported(tile_h, tile_w, dtype, param_dtype))
    return HIMUON_EINVAL;
  if (n_tiles == 0) return 0;
  lds_step_run(params_dev, n_params, tile_begin, n_tiles, tile_h, tile_w, dtype, param_dtype, steps, a, b, c,
               eps, (flags & HIMUON_NS_ROUND_ONCE) != 0, scale_alpha_dev, static_cast<hipStream_t>(stream));
  return (int)hipGetLastError();
}

extern "C" int himuon_ns5_noalloc(uint16_t* x, uint16_t* y, const float* inv, int64_t n_tiles, int mp,
                                  int np, int steps, float a, float b, float c, int flags, void* stream) {
  if (!x || !y || x == y || !inv || n_tiles < 0 || steps < 0 || mp <= 0 || np <= 0 || mp > np ||
      mp % HIMUON_NS_ALIGN || np % HIMUON_NS_ALIGN)
    return HIMUON_EINVAL;
  const size_t per_tile = himuon_ns5_workspace_bytes(1, mp, np);
  if (per_tile > HIMUON_NS_SCRATCH_BYTES) return HIMUON_ENOSPC;  // one tile's A and B do not fit
  if (n_tiles == 0) return 0;
  if (steps == 0)  // no workspace needed
    return himuon_ns5_ex(x, y, inv, n_tiles, mp, np, 0, a, b, c, nullptr, 0, n_tiles, flags, stream);
  int err = 0;
  void* ws = scratch_address(&err);
  if (!ws) return err;
  const int64_t sub_batch = (int64_t)(HIMUON_NS_SCRATCH_BYTES / per_tile);
  return himuon_ns5_ex(x, y, inv, n_tiles, mp, np, steps, a, b, c, ws, HIMUON_NS_SCRATCH_BYTES, sub_batch, flags,
                       stream);
}

extern "C" int himuon_ns5(uint16_t* x, uint16_t* y, const float* inv, int64_t n_tiles, int mp,
                          int np, int steps, float a, float b, float c, void* workspace,
                          size_t workspace_bytes, int64_t sub_batch, void* stream) {
  return himuon_ns5_ex(x, y, inv, n_tiles, mp, np, steps, a, b, c, workspace, workspace_bytes,
                       sub_batch, HIMUON_NS_FAMILY_AUTO, stream);
}

// ---------------------------------------------------------------------------
// The three NS products one at a time (the reference's kernel entry points
// XXT, ba_plus_cAA and fused_bmm_add): contiguous batches, dimensions
// multiples of 128; edges that are multiples of 256 take the stream kernels
// (unless the flags ask for the 128-block family), others the 128-block ones.
// ---------------------------------------------------------------------------
namespace {
bool stage_family(int flags, int* family) {
  *family = flags & HIMUON_NS_FAMILY_MASK;
  return !(flags & ~HIMUON_NS_FAMILY_MASK) &&
         (*family == HIMUON_NS_FAMILY_AUTO || *family == HIMUON_NS_FAMILY_BLOCK128);
}
}  // namespace

extern "C" int himuon_xxt(const uint16_t* x, uint16_t* out, int64_t batch, int M, int K, int flags,
                          void* stream) {
  int family = 0;
  if (!x || !out || batch < 0 || M <= 0 || K <= 0 || M % BM || K % BM || !stage_family(flags, &family))
    return HIMUON_EINVAL;
  if (batch == 0) return 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t xs = (int64_t)M * K, os = (int64_t)M * M;
  if (family == HIMUON_NS_FAMILY_AUTO && M % 256 == 0 && K % 256 == 0) {
    ns_stream_product(0, x, xs, K, x, xs, K, nullptr, 0, 0, out, os, M, M, M, K, batch, 1.f, 0.f, false, s);
  } else {
    const int nb = M / BM;
    hipLaunchKernelGGL(ns_gram_kernel, dim3((unsigned)xcd_grid(batch * (nb * (nb + 1) / 2))), dim3(kThreads), 0,
                       s, x, xs, K, out, os, M, nullptr, M, K, batch, 1.0f, 0.0f);
  }
  return (int)hipGetLastError();
}

extern "C" int himuon_ba_plus_caa(const uint16_t* a, uint16_t* out, int64_t batch, int M, float alpha,
                                  float beta, int flags, void* stream) {
  int family = 0;
  if (!a || !out || a == out || batch < 0 || M <= 0 || M % BM || !stage_family(flags, &family))
    return HIMUON_EINVAL;
  if (batch == 0) return 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t sq = (int64_t)M * M;
  if (family == HIMUON_NS_FAMILY_AUTO && M % 256 == 0) {
    ns_stream_product(1, a, sq, M, a, sq, M, a, sq, M, out, sq, M, M, M, M, batch, alpha, beta, false, s);
  } else {
    const int nb = M / BM;
    hipLaunchKernelGGL(ns_gram_kernel, dim3((unsigned)xcd_grid(batch * (nb * (nb + 1) / 2))), dim3(kThreads), 0,
                       s, a, sq, M, out, sq, M, nullptr, M, M, batch, alpha, beta);
  }
  return (int)hipGetLastError();
}

extern "C" int himuon_bmm_add(const uint16_t* b, const uint16_t* x, uint16_t* out, int64_t batch, int M, int N,
                              float a, int flags, void* stream) {
  int family = 0;
  const bool round_once = (flags & HIMUON_NS_ROUND_ONCE) != 0;
  if (!b || !x || !out || out == x || out == b || batch < 0 || M <= 0 || N <= 0 || M % BM || N % BN ||
      !stage_family(flags & ~HIMUON_NS_ROUND_ONCE, &family))
    return HIMUON_EINVAL;
  if (batch == 0) return 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t sq = (int64_t)M * M, rect = (int64_t)M * N;
  if (family == HIMUON_NS_FAMILY_AUTO && M % 256 == 0 && N % 256 == 0) {
    ns_stream_product(2, b, sq, M, x, rect, N, x, rect, N, out, rect, N, M, N, M, batch, 1.f, a, round_once, s);
  } else {
    hipLaunchKernelGGL(ns_apply_kernel, dim3((unsigned)xcd_grid(batch * (M / BM) * (N / BN))), dim3(kThreads), 0,
                       s, b, sq, x, rect, out, rect, nullptr, M, N, batch, a, round_once ? 1 : 0);
  }
  return (int)hipGetLastError();
}

// ba_plus_cAA followed by fused_bmm_add as one kernel (ns5_ba.hip): B never
// leaves the CU. 512 x 512 only (the fused kernel's tile).
extern "C" int himuon_ba_bmm_add(const uint16_t* a, const uint16_t* x, uint16_t* out, int64_t batch, int M,
                                 int N, float alpha, float beta, float gamma, int flags, void* stream) {
  if (!a || !x || !out || out == x || out == a || batch < 0 || !ns5_ba_supported(M, N) ||
      (flags & ~HIMUON_NS_ROUND_ONCE))
    return HIMUON_EINVAL;
  if (batch == 0) return 0;
  if (!ns5_ba_run(a, x, out, nullptr, batch, gamma, beta, alpha, (flags & HIMUON_NS_ROUND_ONCE) != 0,
                  static_cast<hipStream_t>(stream)))
    return HIMUON_EINVAL;  // batch above kBaMaxTiles (32-bit work-item indices)
  return (int)hipGetLastError();
}
