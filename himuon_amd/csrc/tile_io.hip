// Memory-bound kernels around the Newton-Schulz core:
//   * momentum_gather: Nesterov momentum + zero-padded tile gather into the
//     bf16 NS tile buffer + per-slab sum of squares (himuon.py:350-357,
//     704-719, 239-242).
//   * tile_scale: per-tile 1 / (||X||_F + eps) (himuon.py:242).
//   * untile: NS tile buffer -> per-parameter update (himuon.py:315-329).
// All are HBM-bound: each element is read/written once (14 B/el for fp32
// gather, 6 B/el for fp32 untile), with 16-byte accesses on both sides.
// Plain tiles (tile_h <= tile_w) move whole NS rows: a work item is a slab of
// 32, 64 or 128 NS rows of one tile (16384 elements up to np = 512, whole
// tiles up to 128 x 128), one workgroup per item (2-3 % faster than a
// persistent grid of four workgroups per CU), and each thread issues
// the loads of kVec 8-element vectors before using any of them, so enough
// bytes are in flight to cover the memory latency. Tall tiles are transposed
// through LDS in 64 x 64 blocks.
#include "elem_ops.h"

namespace {

constexpr int kThreads = 256;
constexpr int kSlabElems = 16384;  // NS elements per gather/untile work item (plain tiles)
// 8-element vectors per thread per load batch (untile): with one workgroup
// per slab, 4 (fewer registers, more waves resident) measured 6-7 % faster
// than 8 on bf16 parameters and the same on fp32
constexpr int kVec = 4;
// The plain-tile gather loads grad and momentum vectors: 4 per batch keep it
// at about 150 VGPRs (three workgroups per CU); 8 took all 256 and measured
// 3-6 % slower. Each thread still sums the same elements in the same order.
constexpr int kGatherVec = 4;
constexpr int kBlk = 64;     // NS block edge for the transposed variants
constexpr int kBlkPitch = kBlk + 8;

struct Geo {
  int tile_h, tile_w, mp, np;
};

// NS rows per plain-tile work item: the largest power of two r with
// r * np <= kSlabElems (whole tiles at np = 128), at least 32 and at most mp.
// A power of two no larger than 128 divides mp (a multiple of 128), so the
// slabs cover every row of the padded tile, padding rows included (np = 384
// would give 16384 / 384 = 42 rows otherwise, which leaves rows unwritten).
HM_HD int slab_rows(int mp, int np) {
  int r = 32;
  while (2 * r * np <= kSlabElems && 2 * r <= mp) r *= 2;
  return r;
}

// ---------------------------------------------------------------------------
// Gather, plain tiles: work item = (tile t, slab q of `rows` NS rows, rows =
// slab_rows(mp, np)); NS row i
// of tile (r, c) is parameter row r*tile_h + i, columns c*tile_w + j. Rows and
// columns outside the tile or the parameter are written as zeros. The slab's
// sum of squares of the bf16 values goes to partials[t * (mp / rows) + q].
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(
    const HimuonParamDesc* __restrict__ params, int n_params, int64_t n_tiles, Geo geo,
    uint16_t* __restrict__ tiles, float* __restrict__ partials) {
  __shared__ float red[kThreads / 64];
  const int rows = slab_rows(geo.mp, geo.np);
  const int slabs = geo.mp / rows;
  const int vpr = geo.np / 8;          // 8-element vectors per NS row
  const int per_item = rows * vpr;
  const int64_t total = n_tiles * slabs;
  for (int64_t item = blockIdx.x; item < total; item += gridDim.x) {
    const int64_t t = item / slabs;
    const int q = (int)(item - t * slabs);
    const HimuonParamDesc& P = params[find_param(params, n_params, t)];
    const int64_t lt = t - P.tile0;
    const int r = (int)(lt / P.C), c = (int)(lt % P.C);
    const bool has_mom = P.momentum != nullptr;
    const float mu = P.mu;
    const bool nesterov = P.nesterov != 0;
    uint16_t* out = tiles + t * (int64_t)geo.mp * geo.np;
    float ssq = 0.f;
    for (int v0 = 0; v0 < per_item; v0 += kThreads * kGatherVec) {
      float g[kGatherVec][8], m[kGatherVec][8];
      bool fast[kGatherVec];
      // Phase 1: every load of the batch is issued before any is used.
#pragma unroll
      for (int k = 0; k < kGatherVec; ++k) {
        const int v = v0 + k * kThreads + threadIdx.x;
        const int i = q * rows + v / vpr, j0 = (v % vpr) * 8;
        const int64_t pr = (int64_t)r * geo.tile_h + i, pc = (int64_t)c * geo.tile_w + j0;
        const int64_t og = pr * P.ld_grad + pc, om = pr * P.ld_mom + pc;
        fast[k] = v < per_item && i < geo.tile_h && pr < P.h && j0 + 8 <= geo.tile_w && pc + 8 <= P.w &&
                  aligned16<DT>(P.grad, og) && (!has_mom || aligned16<DT>(P.momentum, om));
        if (fast[k]) {
          load8<DT>(P.grad, og, g[k]);
          if (has_mom) load8<DT>(P.momentum, om, m[k]);
        }
      }
      // Phase 2: momentum, momentum store, bf16 NS operand store.
#pragma unroll
      for (int k = 0; k < kGatherVec; ++k) {
        const int v = v0 + k * kThreads + threadIdx.x;
        if (v >= per_item) continue;
        const int i = q * rows + v / vpr, j0 = (v % vpr) * 8;
        const int64_t pr = (int64_t)r * geo.tile_h + i, pc = (int64_t)c * geo.tile_w + j0;
        const int64_t og = pr * P.ld_grad + pc, om = pr * P.ld_mom + pc;
        float x[8];
        if (fast[k]) {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = momentum_elem<DT>(g[k][e], &m[k][e], mu, nesterov, has_mom);
          if (has_mom) store8<DT>(P.momentum, om, m[k]);
        } else {
          const bool row_ok = i < geo.tile_h && pr < P.h;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            x[e] = 0.f;
            if (row_ok && j0 + e < geo.tile_w && pc + e < P.w) {
              const float gv = load_elem<DT>(P.grad, og + e);
              float mv = has_mom ? load_elem<DT>(P.momentum, om + e) : 0.f;
              x[e] = momentum_elem<DT>(gv, &mv, mu, nesterov, has_mom);
              if (has_mom) store_elem<DT>(P.momentum, om + e, mv);
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
        *reinterpret_cast<uint4*>(out + (int64_t)i * geo.np + j0) =
            make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7]));
      }
    }
    const float sum = block_sum<kThreads>(ssq, red);
    if (threadIdx.x == 0) partials[item] = sum;
    __syncthreads();  // red[] is rewritten by the next item
  }
}

// ---------------------------------------------------------------------------
// Gather, tall tiles (tile_h > tile_w, the NS operand is the tile's
// transpose): work item = (tile, 64x64 block of the NS operand). The block's
// parameter elements are read as 16-byte row segments, momentum is applied,
// and bf16(e) is transposed through LDS into the NS operand.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(kThreads) void gather_trans_kernel(
    const HimuonParamDesc* __restrict__ params, int n_params, int64_t n_tiles, Geo geo,
    uint16_t* __restrict__ tiles, float* __restrict__ partials) {
  __shared__ uint16_t sT[kBlk * kBlkPitch];  // [param col][param row] of the block
  __shared__ float red[kThreads / 64];
  const int bi_n = geo.mp / kBlk, bj_n = geo.np / kBlk;
  const int blocks = bi_n * bj_n;
  const int64_t item = xcd_item(n_tiles * blocks);
  if (item >= n_tiles * blocks) return;
  const int64_t t = item / blocks;
  const int b = (int)(item % blocks);
  const int i0 = (b / bj_n) * kBlk, j0 = (b % bj_n) * kBlk;  // NS block origin
  const int tr0 = j0, tc0 = i0;                                // tile-local origin
  const HimuonParamDesc& P = params[find_param(params, n_params, t)];
  const int64_t lt = t - P.tile0;
  const int r = (int)(lt / P.C), c = (int)(lt % P.C);
  const bool has_mom = P.momentum != nullptr;
  const float mu = P.mu;
  const bool nesterov = P.nesterov != 0;
  uint16_t* ns = tiles + t * (int64_t)geo.mp * geo.np;
  float ssq = 0.f;
  for (int v = threadIdx.x; v < kBlk * (kBlk / 8); v += kThreads) {
    const int rr = v / (kBlk / 8), cv = v % (kBlk / 8);
    const int tr = tr0 + rr, tc = tc0 + cv * 8;
    const int64_t pr = (int64_t)r * geo.tile_h + tr;
    const int64_t pc = (int64_t)c * geo.tile_w + tc;
    const bool row_ok = tr < geo.tile_h && pr < P.h;
    const int64_t og = pr * P.ld_grad + pc, om = pr * P.ld_mom + pc;
    float x[8];
    const bool fast = row_ok && tc + 8 <= geo.tile_w && pc + 8 <= P.w &&
                      aligned16<DT>(P.grad, og) && (!has_mom || aligned16<DT>(P.momentum, om));
    if (fast) {
      float g[8], m[8];
      load8<DT>(P.grad, og, g);
      if (has_mom) load8<DT>(P.momentum, om, m);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = momentum_elem<DT>(g[e], &m[e], mu, nesterov, has_mom);
      if (has_mom) store8<DT>(P.momentum, om, m);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = 0.f;
        if (row_ok && tc + e < geo.tile_w && pc + e < P.w) {
          const float g = load_elem<DT>(P.grad, og + e);
          float m = has_mom ? load_elem<DT>(P.momentum, om + e) : 0.f;
          x[e] = momentum_elem<DT>(g, &m, mu, nesterov, has_mom);
          if (has_mom) store_elem<DT>(P.momentum, om + e, m);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t h = f32_to_bf16(x[e]);
      const float f = bf16_to_f32(h);
      ssq = fmaf(f, f, ssq);
      sT[(cv * 8 + e) * kBlkPitch + rr] = (uint16_t)h;
    }
  }
  __syncthreads();
  for (int v = threadIdx.x; v < kBlk * (kBlk / 8); v += kThreads) {
    const int cc = v / (kBlk / 8), rv = v % (kBlk / 8);
    const uint4 q = *reinterpret_cast<const uint4*>(&sT[cc * kBlkPitch + rv * 8]);
    *reinterpret_cast<uint4*>(ns + (int64_t)(tc0 + cc) * geo.np + tr0 + rv * 8) = q;
  }
  const float s = block_sum<kThreads>(ssq, red);
  if (threadIdx.x == 0) partials[t * blocks + b] = s;
}

__global__ __launch_bounds__(kThreads) void tile_scale_kernel(const float* __restrict__ partials,
                                                             int per_tile, int64_t n_tiles,
                                                             float eps, float* __restrict__ inv) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= n_tiles) return;
  float s = 0.f;
  for (int q = 0; q < per_tile; ++q) s += partials[t * per_tile + q];
  inv[t] = 1.0f / (sqrtf(s) + eps);
}

// ---------------------------------------------------------------------------
// Untile, plain tiles: update[pr, pc] = scale * NS(i, j). Work item = (tile,
// slab of `rows` NS rows); only NS columns < tile_w hold data.
// ---------------------------------------------------------------------------
template <bool APPLY, int DT>
__global__ __launch_bounds__(kThreads) void untile_rows_kernel(
    const HimuonParamDesc* __restrict__ params, int n_params, int64_t n_tiles, Geo geo,
    const uint16_t* __restrict__ tiles, const float* __restrict__ sa) {
  const int rows = slab_rows(geo.mp, geo.np);
  const int slabs = geo.mp / rows;
  const int vcols = (geo.tile_w + 7) / 8;
  const int per_item = rows * vcols;
  const int64_t total = n_tiles * slabs;
  for (int64_t item = blockIdx.x; item < total; item += gridDim.x) {
    const int64_t t = item / slabs;
    const int q = (int)(item - t * slabs);
    const HimuonParamDesc& P = params[find_param(params, n_params, t)];
    const int64_t lt = t - P.tile0;
    const int r = (int)(lt / P.C), c = (int)(lt % P.C);
    const float sc = P.upd_scale;
    const uint16_t* in = tiles + t * (int64_t)geo.mp * geo.np;
    for (int v0 = 0; v0 < per_item; v0 += kThreads * kVec) {
      uint4 qv[kVec];
      bool ok[kVec];
#pragma unroll
      for (int k = 0; k < kVec; ++k) {
        const int v = v0 + k * kThreads + threadIdx.x;
        const int i = q * rows + v / vcols, j0 = (v % vcols) * 8;
        const int64_t pr = (int64_t)r * geo.tile_h + i, pc = (int64_t)c * geo.tile_w + j0;
        ok[k] = v < per_item && i < geo.tile_h && pr < P.h && pc < P.w;
        if (ok[k]) qv[k] = *reinterpret_cast<const uint4*>(in + (int64_t)i * geo.np + j0);
      }
#pragma unroll
      for (int k = 0; k < kVec; ++k) {
        if (!ok[k]) continue;
        const int v = v0 + k * kThreads + threadIdx.x;
        const int i = q * rows + v / vcols, j0 = (v % vcols) * 8;
        const int64_t pr = (int64_t)r * geo.tile_h + i, pc = (int64_t)c * geo.tile_w + j0;
        const uint32_t w[4] = {qv[k].x, qv[k].y, qv[k].z, qv[k].w};
        float y[8];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          y[2 * e2] = sc * bf16_to_f32(w[e2] & 0xffffu);
          y[2 * e2 + 1] = sc * __uint_as_float(w[e2] & 0xffff0000u);
        }
        const int64_t ou = pr * P.ld_upd + pc;
        const bool full = j0 + 8 <= geo.tile_w && pc + 8 <= P.w && aligned16<DT>(P.update, ou);
        const int valid = (int)min<int64_t>(min(8, geo.tile_w - j0), P.w - pc);
        put8<APPLY, DT>(P, ou, y, full, valid, sa);
      }
    }
  }
}

// Untile, transposed tiles: update[pr, pc] = scale * NS(pc_local, pr_local).
template <bool APPLY, int DT>
__global__ __launch_bounds__(kThreads) void untile_trans_kernel(
    const HimuonParamDesc* __restrict__ params, int n_params, int64_t n_tiles, Geo geo,
    const uint16_t* __restrict__ tiles, const float* __restrict__ sa) {
  __shared__ uint16_t sT[kBlk * kBlkPitch];  // [tile row tr][tile col tc]
  const int bi_n = geo.mp / kBlk, bj_n = geo.np / kBlk;
  const int blocks = bi_n * bj_n;
  const int64_t item = xcd_item(n_tiles * blocks);
  if (item >= n_tiles * blocks) return;
  const int64_t t = item / blocks;
  const int b = (int)(item % blocks);
  const int i0 = (b / bj_n) * kBlk, j0 = (b % bj_n) * kBlk;
  // NS rows i0.. are tile cols; NS cols j0.. are tile rows. Skip pure padding.
  if (i0 >= geo.tile_w || j0 >= geo.tile_h) return;
  const HimuonParamDesc& P = params[find_param(params, n_params, t)];
  const int64_t lt = t - P.tile0;
  const int r = (int)(lt / P.C), c = (int)(lt % P.C);
  const uint16_t* in = tiles + t * (int64_t)geo.mp * geo.np;
  for (int v = threadIdx.x; v < kBlk * (kBlk / 8); v += kThreads) {
    const int ii = v / (kBlk / 8), jv = v % (kBlk / 8);
    const uint4 q = *reinterpret_cast<const uint4*>(in + (int64_t)(i0 + ii) * geo.np + j0 + jv * 8);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      sT[(jv * 8 + 2 * k) * kBlkPitch + ii] = (uint16_t)(w[k] & 0xffffu);
      sT[(jv * 8 + 2 * k + 1) * kBlkPitch + ii] = (uint16_t)(w[k] >> 16);
    }
  }
  __syncthreads();
  const float sc = P.upd_scale;
  for (int v = threadIdx.x; v < kBlk * (kBlk / 8); v += kThreads) {
    const int rr = v / (kBlk / 8), cv = v % (kBlk / 8);
    const int tr = j0 + rr, tc = i0 + cv * 8;
    const int64_t pr = (int64_t)r * geo.tile_h + tr;
    const int64_t pc = (int64_t)c * geo.tile_w + tc;
    if (tr >= geo.tile_h || pr >= P.h || tc >= geo.tile_w || pc >= P.w) continue;
    const uint4 q = *reinterpret_cast<const uint4*>(&sT[rr * kBlkPitch + cv * 8]);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float y[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      y[2 * k] = sc * bf16_to_f32(w[k] & 0xffffu);
      y[2 * k + 1] = sc * __uint_as_float(w[k] & 0xffff0000u);
    }
    const int64_t ou = pr * P.ld_upd + pc;
    const bool full = tc + 8 <= geo.tile_w && pc + 8 <= P.w && aligned16<DT>(P.update, ou);
    const int valid = (int)min<int64_t>(min(8, geo.tile_w - tc), P.w - pc);
    put8<APPLY, DT>(P, ou, y, full, valid, sa);
  }
}

int num_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

bool geo_ok(int tile_h, int tile_w, int mp, int np) {
  const int m = tile_h <= tile_w ? tile_h : tile_w;
  const int n = tile_h <= tile_w ? tile_w : tile_h;
  return tile_h > 0 && tile_w > 0 && mp >= m && np >= n && mp % HIMUON_NS_ALIGN == 0 &&
         np % HIMUON_NS_ALIGN == 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int himuon_gather_partials_per_tile(int tile_h, int tile_w, int mp, int np) {
  if (!geo_ok(tile_h, tile_w, mp, np)) return HIMUON_EINVAL;
  return tile_h > tile_w ? (mp / kBlk) * (np / kBlk) : mp / slab_rows(mp, np);
}

extern "C" int himuon_momentum_gather(const HimuonParamDesc* params_dev, int n_params,
                                      int64_t n_tiles, int tile_h, int tile_w, int mp, int np,
                                      int dtype, uint16_t* tiles_bf16, float* partials,
                                      void* stream) {
  if (!geo_ok(tile_h, tile_w, mp, np) || n_params <= 0 || n_tiles < 0 || !params_dev ||
      !tiles_bf16 || !partials)
    return HIMUON_EINVAL;
  if (n_tiles == 0) return 0;
  const Geo geo{tile_h, tile_w, mp, np};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t items = n_tiles * himuon_gather_partials_per_tile(tile_h, tile_w, mp, np);
  const dim3 block(kThreads);
  if (tile_h > tile_w) {
    const dim3 grid((unsigned)xcd_grid(items));
    switch (dtype) {
      case HIMUON_DTYPE_F32: hipLaunchKernelGGL(gather_trans_kernel<HIMUON_DTYPE_F32>, grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, partials); break;
      case HIMUON_DTYPE_BF16: hipLaunchKernelGGL(gather_trans_kernel<HIMUON_DTYPE_BF16>, grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, partials); break;
      case HIMUON_DTYPE_F16: hipLaunchKernelGGL(gather_trans_kernel<HIMUON_DTYPE_F16>, grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, partials); break;
      default: return HIMUON_EINVAL;
    }
  } else {
    const dim3 grid((unsigned)std::min<int64_t>(items, (int64_t)1 << 30));
    switch (dtype) {
      case HIMUON_DTYPE_F32: hipLaunchKernelGGL(gather_rows_kernel<HIMUON_DTYPE_F32>, grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, partials); break;
      case HIMUON_DTYPE_BF16: hipLaunchKernelGGL(gather_rows_kernel<HIMUON_DTYPE_BF16>, grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, partials); break;
      case HIMUON_DTYPE_F16: hipLaunchKernelGGL(gather_rows_kernel<HIMUON_DTYPE_F16>, grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, partials); break;
      default: return HIMUON_EINVAL;
    }
  }
  return (int)hipGetLastError();
}

extern "C" int himuon_tile_scale(const float* partials, int partials_per_tile, int64_t n_tiles,
                                 float eps, float* inv, void* stream) {
  if (!partials || !inv || partials_per_tile <= 0 || n_tiles < 0) return HIMUON_EINVAL;
  if (n_tiles == 0) return 0;
  const dim3 grid((unsigned)((n_tiles + kThreads - 1) / kThreads)), block(kThreads);
  hipLaunchKernelGGL(tile_scale_kernel, grid, block, 0, static_cast<hipStream_t>(stream),
                     partials, partials_per_tile, n_tiles, eps, inv);
  return (int)hipGetLastError();
}

namespace {
template <bool APPLY>
int untile_launch(const HimuonParamDesc* params_dev, int n_params, int64_t n_tiles, int tile_h, int tile_w,
                  int mp, int np, int dtype, const uint16_t* tiles_bf16, const float* sa, void* stream) {
  if (!geo_ok(tile_h, tile_w, mp, np) || n_params <= 0 || n_tiles < 0 || !params_dev || !tiles_bf16)
    return HIMUON_EINVAL;
  if (n_tiles == 0) return 0;
  const Geo geo{tile_h, tile_w, mp, np};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 block(kThreads);
  if (tile_h > tile_w) {
    const dim3 grid((unsigned)xcd_grid(n_tiles * (mp / kBlk) * (np / kBlk)));
    switch (dtype) {
      case HIMUON_DTYPE_F32: hipLaunchKernelGGL((untile_trans_kernel<APPLY, HIMUON_DTYPE_F32>), grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, sa); break;
      case HIMUON_DTYPE_BF16: hipLaunchKernelGGL((untile_trans_kernel<APPLY, HIMUON_DTYPE_BF16>), grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, sa); break;
      case HIMUON_DTYPE_F16: hipLaunchKernelGGL((untile_trans_kernel<APPLY, HIMUON_DTYPE_F16>), grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, sa); break;
      default: return HIMUON_EINVAL;
    }
  } else {
    const dim3 grid((unsigned)std::min<int64_t>(n_tiles * (mp / slab_rows(mp, np)), (int64_t)1 << 30));
    switch (dtype) {
      case HIMUON_DTYPE_F32: hipLaunchKernelGGL((untile_rows_kernel<APPLY, HIMUON_DTYPE_F32>), grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, sa); break;
      case HIMUON_DTYPE_BF16: hipLaunchKernelGGL((untile_rows_kernel<APPLY, HIMUON_DTYPE_BF16>), grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, sa); break;
      case HIMUON_DTYPE_F16: hipLaunchKernelGGL((untile_rows_kernel<APPLY, HIMUON_DTYPE_F16>), grid, block, 0, s, params_dev, n_params, n_tiles, geo, tiles_bf16, sa); break;
      default: return HIMUON_EINVAL;
    }
  }
  return (int)hipGetLastError();
}
}  // namespace

extern "C" int himuon_untile(const HimuonParamDesc* params_dev, int n_params, int64_t n_tiles,
                             int tile_h, int tile_w, int mp, int np, int dtype,
                             const uint16_t* tiles_bf16, void* stream) {
  return untile_launch<false>(params_dev, n_params, n_tiles, tile_h, tile_w, mp, np, dtype, tiles_bf16,
                              nullptr, stream);
}

extern "C" int himuon_untile_apply(const HimuonParamDesc* params_dev, int n_params, int64_t n_tiles,
                                   int tile_h, int tile_w, int mp, int np, int param_dtype,
                                   const uint16_t* tiles_bf16, const float* scale_alpha_dev,
                                   void* stream) {
  if (!scale_alpha_dev) return HIMUON_EINVAL;
  return untile_launch<true>(params_dev, n_params, n_tiles, tile_h, tile_w, mp, np, param_dtype, tiles_bf16,
                             scale_alpha_dev, stream);
}
