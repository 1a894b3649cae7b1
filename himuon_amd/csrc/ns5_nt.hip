// Persistent NT-GEMM for the three NS5 stages on 256x256 output blocks
// (NS tiles whose padded edges are multiples of 256).
//
// Every stage is C = epilogue(P Q^T) with P and Q row-major and contracted
// along their rows:
//   GramA : P = Q = X (K = n)          C = A = bf16(X X^T)           (lower blocks)
//   GramB : P = Q = A (K = m)          C = B = bf16(c A A^T + b A)   (lower blocks)
//   Apply : P = B, Q = X^T (K = m)     C = X' = bf16(bf16(B X) + a X), also X'^T
// (ns5_smem.py:89-101, XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88).
// Keeping X in both orientations (a prep pass writes X0 = bf16(x * inv) and
// X0^T, each Apply writes X'^T) makes all three stages the same k-contiguous
// NT product.
//
// Work distribution: a persistent grid (one 256-thread workgroup per CU);
// workgroup w of XCD x (w = blockIdx/8, x = blockIdx%8) walks the items
// ibeg(x) + w, + 32, ... so the blocks of one NS tile run on one XCD and
// share its L2. Per block, K is streamed in 64-wide slabs straight from
// global memory into LDS (global_load_lds_dwordx4, two LDS stages: the next
// slab loads while the current one is multiplied), so no registers stage the
// operands. A slab panel is 256 rows x 128 B with the 16-byte chunks of row r
// stored at position chunk ^ (r & 7): the loader picks the source chunk per
// lane (the LDS destination of a direct load is fixed: lane l writes bytes
// 16l..16l+15 of the wave's 1 KiB), and the MFMA fragment reads of 8
// consecutive rows then hit 8 distinct bank groups. 4 waves in 2x2, each a
// 128x128 sub-block of 4x4 v_mfma_f32_32x32x16_bf16 tiles with swapped
// operands, so lane l holds C[row l%32][4 consecutive columns]: 8-byte
// row-segment stores. Mirrored (GramA/B off-diagonal) and transposed (Apply)
// outputs go through a 128-row LDS image (aliasing the stage buffers) in two
// passes.
#include "ns5_kernels.h"

namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) const u32x4_t lds_u32x4;
typedef __attribute__((address_space(1))) const void gbl_void;

constexpr int NT = 256;
constexpr int BT = 256;                      // output block edge
constexpr int BK = 64;                       // K slab (elements) = 128 B per row
constexpr int PANEL_BYTES = BT * BK * 2;     // one operand slab: 32 KiB
constexpr int STAGE_BYTES = 2 * PANEL_BYTES; // P and Q slabs
constexpr int LDS_BYTES = 2 * STAGE_BYTES;   // two stages: 128 KiB
constexpr int IMGR = 128;                    // image rows per pass
constexpr int LDI = BT + 8;                  // image pitch (elements)
static_assert(IMGR * LDI * 2 <= LDS_BYTES, "image must fit in the stage buffers");

enum { kGramA = 0, kGramB = 1, kApply = 2 };

struct NtArgs {
  const uint16_t* P; int64_t p_bs; int ldp;    // rows i (output rows)
  const uint16_t* Q; int64_t q_bs; int ldq;    // rows j (output columns)
  const uint16_t* R; int64_t r_bs; int ldr;    // epilogue operand [i][j] (A or X)
  uint16_t* C; int64_t c_bs; int ldc;          // output [i][j]
  uint16_t* CT; int64_t ct_bs; int ldct;       // Apply: transposed output [j][i] (or null)
  int M, N, K;
  int64_t ntiles;
  float alpha, beta;                           // Gram: alpha*PQ^T + beta*R; Apply: beta = a
};

HM_DEV f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima): this wave's
// direct-to-LDS loads have landed.
HM_DEV void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// s_waitcnt lgkmcnt(0) (vmcnt and expcnt left at their maxima).
HM_DEV void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// One 256x256 output block: C[tile][bi-block][bj-block]. Kept out of line:
// inlined into the persistent item loop, the register allocator spills.
template <int MODE>
__device__ __noinline__ void nt_item(const NtArgs& g, lds_u8* lds, int64_t tile, int bi, int bj) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  const int nk = g.K / BK;

  // Loader: load i of wave w fills rows 32i + 8w .. +7 of a slab panel; lane
  // l lands at row 8w + 32i + l/8, position l%8, so it reads source chunk
  // (l%8) ^ (l/8) of that row.
  const int lr = lane >> 3, lc = (lane & 7) ^ lr;
  const uint16_t* psrc = g.P + tile * g.p_bs + (int64_t)(bi * BT + 8 * wave + lr) * g.ldp + lc * 8;
  const uint16_t* qsrc = g.Q + tile * g.q_bs + (int64_t)(bj * BT + 8 * wave + lr) * g.ldq + lc * 8;
  const int64_t pstep = 32 * (int64_t)g.ldp, qstep = 32 * (int64_t)g.ldq;
  lds_u8* const wdst = lds + wave * 1024;
  auto issue = [&](int kt, int st) {
    lds_u8* d = wdst + st * STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_global_load_lds((gbl_void*)(psrc + i * pstep + kt * BK), d + i * 4096, 16, 0, 0);
      __builtin_amdgcn_global_load_lds((gbl_void*)(qsrc + i * qstep + kt * BK),
                                       d + PANEL_BYTES + i * 4096, 16, 0, 0);
    }
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  // MFMA fragments of sub-step ks: lane reads row l32 of a 32-row fragment,
  // k-chunk 2 ks + hi, stored at position (2 ks + hi) ^ (l32 & 7). A operand =
  // rows j (Q, columns of C), B operand = rows i (P); the next sub-step's
  // fragments load during the current sub-step's MFMAs.
  const int qrow = (wn * 128 + l32) * 128, prow = (wm * 128 + l32) * 128;
  auto frags = [&](int st, int ks, u32x4_t(&fa)[4], u32x4_t(&fb)[4]) {
    const lds_u8* ps = lds + st * STAGE_BYTES;
    const lds_u8* qs = ps + PANEL_BYTES;
    const int pos = ((2 * ks + hi) ^ (l32 & 7)) * 16;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      fa[t] = *reinterpret_cast<lds_u32x4*>(qs + qrow + t * 4096 + pos);
      fb[t] = *reinterpret_cast<lds_u32x4*>(ps + prow + t * 4096 + pos);
    }
  };
  // One slab from stage st: the 8 fragment reads of sub-step ks + 1 are
  // issued ahead of sub-step ks's 16 MFMAs (sched_barrier fences keep the
  // scheduler from sinking each read next to its MFMA and waiting on it);
  // with LOAD, slab ktn's 16 direct loads into the other stage are
  // interleaved one per MFMA of the first sub-step.
  constexpr int kMfma = 0x008, kVmem = 0x010;
  auto slab = [&](auto load_tag, int st, int ktn) {
    constexpr bool LOAD = decltype(load_tag)::value;
    u32x4_t fa[2][4], fb[2][4];
    frags(st, 0, fa[0], fb[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      // Sub-step ks's reads have landed (they had the previous 16 MFMAs to do
      // so). Waiting here keeps at most 8 LDS reads in flight: past the 15
      // the lgkmcnt field can count, the compiler waits for all of them.
      wait_lgkm0();
      if (ks + 1 < BK / 16) frags(st, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      if (LOAD && ks == 0) issue(ktn, st ^ 1);
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
          acc[tj][ti] = mfma(fa[ks & 1][tj], fb[ks & 1][ti], acc[tj][ti]);
      if (LOAD && ks == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kVmem, 1, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using kLoad = std::integral_constant<bool, true>;
  using kNoLoad = std::integral_constant<bool, false>;

  // Slab kt + 1 loads into the other stage while slab kt is multiplied; the
  // barrier after each wave's vmcnt(0) publishes slab kt to every wave and
  // tells the loader that slab kt - 1's stage is free again. nk is even (K is
  // a multiple of 256) and the last pair is peeled, so the MFMAs sit in
  // straight-line code: a conditional around them makes the register
  // allocator shuttle the accumulators between AGPRs and VGPRs.
  __syncthreads();  // the previous item's last reads of the stage buffers are done
  issue(0, 0);
  wait_vm0();
  __syncthreads();
  for (int kt = 0; kt < nk - 2; kt += 2) {
    slab(kLoad{}, 0, kt + 1);
    wait_vm0();
    __syncthreads();
    slab(kLoad{}, 1, kt + 2);
    wait_vm0();
    __syncthreads();
  }
  slab(kLoad{}, 0, nk - 1);
  wait_vm0();
  __syncthreads();
  slab(kNoLoad{}, 1, 0);
  __syncthreads();  // all waves are done with the stage buffers (the image reuses them)

  // Epilogue. Lane holds C[i][j..j+3], i = row0 + l32, j = col0 + 8q + 4hi.
  // The R operand (A or X) of all 64 groups is loaded before any store: a
  // load issued after stores would wait for them (in-order vmcnt).
  __attribute__((address_space(3))) uint16_t* const img =
      reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(lds);
  u32x2_t rvals[4][4][4];
  if constexpr (MODE != kGramA) {
    const uint16_t* rb = g.R + tile * g.r_bs;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int i = bi * BT + wm * 128 + ti * 32 + l32;
          const int j = bj * BT + wn * 128 + tj * 32 + 8 * q + 4 * hi;
          rvals[ti][tj][q] = *reinterpret_cast<const u32x2_t*>(rb + (int64_t)i * g.ldr + j);
        }
  }
  auto outvals = [&](int ti, int tj, int q, uint32_t(&h)[4]) {
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = acc[tj][ti][4 * q + e];
    if constexpr (MODE == kGramA) {
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = f32_to_bf16(g.alpha * v[e]);
    } else {
      const u32x2_t rv = rvals[ti][tj][q];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = bf16_to_f32(half16(rv[e >> 1], e & 1));
        if constexpr (MODE == kApply)
          h[e] = f32_to_bf16(fmaf(g.beta, x, round_bf16(v[e])));
        else
          h[e] = f32_to_bf16(fmaf(g.beta, x, g.alpha * v[e]));
      }
    }
  };

  const bool image = (MODE == kApply) ? (g.CT != nullptr) : (bi != bj);
  uint16_t* Ct = g.C + tile * g.c_bs;
  // Pass 0: every lane stores its row segments; waves with wn == 0 also
  // write their half of the transposed image.
#pragma unroll
  for (int ti = 0; ti < 4; ++ti)
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t h[4];
        outvals(ti, tj, q, h);
        const int il = wm * 128 + ti * 32 + l32;
        const int jl = wn * 128 + tj * 32 + 8 * q + 4 * hi;
        u32x2_t o;
        o[0] = pack2(h[0], h[1]);
        o[1] = pack2(h[2], h[3]);
        *reinterpret_cast<u32x2_t*>(Ct + (int64_t)(bi * BT + il) * g.ldc + bj * BT + jl) = o;
        if (image && wn == 0) {
#pragma unroll
          for (int e = 0; e < 4; ++e) img[(jl + e) * LDI + il] = (uint16_t)h[e];
        }
      }
  if (!image) return;
  uint16_t* Dt = (MODE == kApply) ? g.CT + tile * g.ct_bs : Ct;
  const int ldd = (MODE == kApply) ? g.ldct : g.ldc;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1 && wn == 1) {
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int tj = 0; tj < 4; ++tj)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint32_t h[4];
            outvals(ti, tj, q, h);
            const int il = wm * 128 + ti * 32 + l32;
            const int jl = tj * 32 + 8 * q + 4 * hi;  // within this pass's 128 rows
#pragma unroll
            for (int e = 0; e < 4; ++e) img[(jl + e) * LDI + il] = (uint16_t)h[e];
          }
    }
    __syncthreads();
    // Image row r = output column bj*256 + pass*128 + r -> a row of the
    // transposed / mirrored block.
    for (int v = tid; v < IMGR * (BT / 8); v += NT) {
      const int r = v >> 5, c8 = (v & 31) * 8;
      const u32x4_t val = *reinterpret_cast<lds_u32x4*>(img + r * LDI + c8);
      *reinterpret_cast<u32x4_t*>(Dt + (int64_t)(bj * BT + pass * IMGR + r) * ldd + bi * BT + c8) =
          val;
    }
    __syncthreads();
  }
}

template <int MODE>
__global__ __launch_bounds__(NT, 1) void ns_nt_kernel(NtArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
  const int nbi = g.M / BT, nbj = g.N / BT;
  const int per_tile = (MODE == kApply) ? nbi * nbj : nbi * (nbi + 1) / 2;
  const int64_t total = g.ntiles * per_tile;
  const int wper = (int)(gridDim.x >> 3);
  const int64_t per_xcd = (total + 7) >> 3;
  const int64_t ibeg = (int64_t)(blockIdx.x & 7) * per_xcd;
  const int64_t iend = (ibeg + per_xcd < total) ? ibeg + per_xcd : total;
  for (int64_t item = ibeg + (blockIdx.x >> 3); item < iend; item += wper) {
    const int64_t tile = item / per_tile;
    const int p = (int)(item - tile * per_tile);
    int bi, bj;
    if (MODE == kApply) {
      bi = p / nbj;
      bj = p - bi * nbj;
    } else {
      bi = 0;
      while ((bi + 1) * (bi + 2) / 2 <= p) ++bi;
      bj = p - bi * (bi + 1) / 2;
    }
    nt_item<MODE>(g, (lds_u8*)lds, tile, bi, bj);
  }
}

// X0 = bf16(x * inv) in place and X0^T, one 64x64 block per workgroup.
__global__ __launch_bounds__(NT) void ns_nt_prep_kernel(uint16_t* __restrict__ x,
                                                        uint16_t* __restrict__ xt,
                                                        const float* __restrict__ inv, int mp,
                                                        int np, int64_t ntiles) {
  __shared__ uint16_t blk[64][66];
  const int nbr = mp / 64, nbc = np / 64;
  const int64_t item = xcd_item(ntiles * nbr * nbc);
  if (item >= ntiles * nbr * nbc) return;
  const int64_t tile = item / (nbr * nbc);
  const int p = (int)(item - tile * nbr * nbc);
  const int br = p / nbc, bc = p - br * nbc;
  const float s = inv[tile];
  const int t = threadIdx.x;
  {
    const int r = t >> 2, c0 = (t & 3) * 16;
    uint16_t* src = x + tile * (int64_t)mp * np + (int64_t)(br * 64 + r) * np + bc * 64 + c0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4_t v = scale8(reinterpret_cast<const u32x4_t*>(src)[h], s);
      reinterpret_cast<u32x4_t*>(src)[h] = v;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        blk[r][c0 + 8 * h + 2 * k] = (uint16_t)(v[k] & 0xffffu);
        blk[r][c0 + 8 * h + 2 * k + 1] = (uint16_t)(v[k] >> 16);
      }
    }
  }
  __syncthreads();
  {
    const int c = t >> 2, r0 = (t & 3) * 16;
    uint16_t* dst = xt + tile * (int64_t)mp * np + (int64_t)(bc * 64 + c) * mp + br * 64 + r0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4_t v;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        v[k] = pack2(blk[r0 + 8 * h + 2 * k][c], blk[r0 + 8 * h + 2 * k + 1][c]);
      reinterpret_cast<u32x4_t*>(dst)[h] = v;
    }
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
void launch(const NtArgs& a, int64_t items, hipStream_t s) {
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t wgs_per_xcd = std::max<int64_t>(1, std::min<int64_t>(num_cus() / 8, per_xcd));
  hipLaunchKernelGGL((ns_nt_kernel<MODE>), dim3((unsigned)(8 * wgs_per_xcd)), dim3(NT), 0, s, a);
}

}  // namespace

bool ns5_nt_supported(int mp, int np) { return mp % BT == 0 && np % BT == 0; }

// One sub-batch of `cnt` tiles, `steps` >= 1 iterations, ping-ponging X
// between (x, xt) and (y, yt); A and B live in the workspace. x is scaled in
// place (X0) and xt receives X0^T first, so the caller's xt content is unused.
void ns5_nt_run(uint16_t* x, uint16_t* xt, uint16_t* y, uint16_t* yt, const float* inv,
                int64_t cnt, int mp, int np, int steps, float a, float b, float c, uint16_t* wsA,
                uint16_t* wsB, hipStream_t s) {
  const int64_t sq = (int64_t)mp * mp, rect = (int64_t)mp * np;
  const int nb = mp / BT;
  const int64_t gram_items = cnt * (nb * (nb + 1) / 2);
  const int64_t apply_items = cnt * nb * (np / BT);
  const int64_t prep_items = cnt * (mp / 64) * (np / 64);
  hipLaunchKernelGGL(ns_nt_prep_kernel, dim3((unsigned)xcd_grid(prep_items)), dim3(NT), 0, s, x,
                     xt, inv, mp, np, cnt);
  uint16_t* cur = x;
  uint16_t* curT = xt;
  uint16_t* nxt = y;
  uint16_t* nxtT = yt;
  for (int it = 0; it < steps; ++it) {
    const bool last = it == steps - 1;
    const NtArgs ga{cur, rect, np, cur, rect, np, nullptr, 0, 0, wsA, sq, mp, nullptr, 0, 0,
                    mp, mp, np, cnt, 1.0f, 0.0f};
    launch<kGramA>(ga, gram_items, s);
    const NtArgs gb{wsA, sq, mp, wsA, sq, mp, wsA, sq, mp, wsB, sq, mp, nullptr, 0, 0,
                    mp, mp, mp, cnt, c, b};
    launch<kGramB>(gb, gram_items, s);
    const NtArgs ap{wsB, sq, mp, curT, rect, mp, cur, rect, np, nxt, rect, np,
                    last ? nullptr : nxtT, rect, mp, mp, np, mp, cnt, 1.0f, a};
    launch<kApply>(ap, apply_items, s);
    std::swap(cur, nxt);
    std::swap(curT, nxtT);
  }
}
