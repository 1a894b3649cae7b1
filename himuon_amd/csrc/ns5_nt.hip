// Persistent NT-GEMM for the three NS5 stages on 256x256 output blocks
// (NS tiles whose padded edges are multiples of 256).
//
// Every stage is C = epilogue(P Q^T) with P and Q row-major and contracted
// along their rows:
//   GramA : P = Q = X (K = n)          C = A = bf16(X X^T)           (lower blocks)
//   GramB : P = Q = A (K = m)          C = B = bf16(c A A^T + b A)   (lower blocks)
//   Apply : P = B, Q = X^T (K = m)     C = X' = bf16(bf16(B X) + a X), also X'^T
// (ns5_smem.py:89-101, XXT.py:55-75, ba_plus_cAA.py:58-85, fused_bmm_add.py:65-88).
// Keeping X in both orientations (the gather writes X0^T, each Apply writes
// X'^T) makes all three stages the same k-contiguous NT product.
//
// Work distribution: a persistent grid (one 256-thread workgroup per CU);
// workgroup w of XCD x (w = blockIdx/8, x = blockIdx%8) walks the items
// ibeg(x) + w, + 32, ... so the blocks of one NS tile run on one XCD and
// share its L2. Per block, K is streamed in 64-wide slabs through registers
// (two slabs in flight) into two padded LDS stages; MFMA fragment reads of the
// next 16-wide sub-step overlap the current sub-step's MFMAs. 4 waves in 2x2, each a 128x128 sub-block of 4x4
// v_mfma_f32_32x32x16_bf16 tiles with swapped operands, so lane l holds
// C[row l%32][4 consecutive columns]: 8-byte row-segment stores. Mirrored
// (GramA/B off-diagonal) and transposed (Apply) outputs go through a 128-row
// LDS image (aliasing the stage buffers) in two passes.
#include "ns5_kernels.h"

namespace {

constexpr int NT = 256;
constexpr int BT = 256;           // output block edge
constexpr int BK = 64;            // K slab
constexpr int LDK = BK + 8;       // padded LDS row pitch (elements)
constexpr int PANEL = BT * LDK;   // elements per staged operand panel
constexpr int DEPTH = 2;          // K slabs in flight in registers
constexpr int CH = BT * BK / 8 / NT;  // 16-byte chunks per thread per panel (8)
constexpr int RPT = NT / (BK / 8);    // rows covered per loader pass (32)
constexpr int IMGR = 128;         // image rows per pass
constexpr int LDI = BT + 8;       // image pitch
constexpr int LDS_ELEMS = 4 * PANEL;  // two stages of (P, Q); the image aliases them
static_assert(IMGR * LDI <= LDS_ELEMS, "image must fit in the stage buffers");

enum { kGramA = 0, kGramB = 1, kApply = 2 };

struct NtArgs {
  const uint16_t* P; int64_t p_bs; int ldp;    // rows i (output rows)
  const uint16_t* Q; int64_t q_bs; int ldq;    // rows j (output columns)
  const uint16_t* R; int64_t r_bs; int ldr;    // epilogue operand [i][j] (A or X)
  uint16_t* C; int64_t c_bs; int ldc;          // output [i][j]
  uint16_t* CT; int64_t ct_bs; int ldct;       // Apply: transposed output [j][i] (or null)
  const float* inv;                            // per-tile normaliser (SCALED)
  int M, N, K;
  int64_t ntiles;
  float alpha, beta;                           // Gram: alpha*PQ^T + beta*R; Apply: beta = a
};

HM_DEV f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// One 256x256 output block: C[tile][bi-block][bj-block]. Kept out of line:
// inlined into the persistent item loop, the register allocator spills.
template <int MODE, bool SCALED>
__device__ __noinline__ void nt_item(const NtArgs& g, uint16_t* lds, int64_t tile, int bi, int bj) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  const int lrow = tid / (BK / 8), lkc = (tid % (BK / 8)) * 8;  // loader: rows lrow + RPT*q
  const int nk = g.K / BK;
  const float sc = SCALED ? g.inv[tile] : 1.f;

  const uint16_t* pbase = g.P + tile * g.p_bs + (int64_t)(bi * BT + lrow) * g.ldp + lkc;
  const uint16_t* qbase = g.Q + tile * g.q_bs + (int64_t)(bj * BT + lrow) * g.ldq + lkc;
  const int64_t pstep = (int64_t)RPT * g.ldp, qstep = (int64_t)RPT * g.ldq;

  auto issue = [&](int kt, u32x4_t(&r)[2 * CH]) {
    const uint16_t* p = pbase + kt * BK;
    const uint16_t* q = qbase + kt * BK;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      r[i] = *reinterpret_cast<const u32x4_t*>(p + i * pstep);
      r[CH + i] = *reinterpret_cast<const u32x4_t*>(q + i * qstep);
    }
  };
  auto stage_in = [&](const u32x4_t(&r)[2 * CH], int st) {
    uint16_t* ps = lds + st * 2 * PANEL;
    uint16_t* qs = ps + PANEL;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int off = (lrow + RPT * i) * LDK + lkc;
      const u32x4_t pv = (SCALED && MODE == kGramA) ? scale8(r[i], sc) : r[i];
      const u32x4_t qv = (SCALED && MODE != kGramB) ? scale8(r[CH + i], sc) : r[CH + i];
      *reinterpret_cast<u32x4_t*>(ps + off) = pv;
      *reinterpret_cast<u32x4_t*>(qs + off) = qv;
    }
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  // MFMA fragments of sub-step ks: A operand = rows j (columns of C), B
  // operand = rows i; the next sub-step's fragments load during the MFMAs.
  auto frags = [&](int st, int ks, u32x4_t(&fa)[4], u32x4_t(&fb)[4]) {
    const uint16_t* ps = lds + st * 2 * PANEL;
    const uint16_t* qs = ps + PANEL;
    const int kk = ks * 16 + hi * 8;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      fa[t] = *reinterpret_cast<const u32x4_t*>(qs + (wn * 128 + t * 32 + l32) * LDK + kk);
      fb[t] = *reinterpret_cast<const u32x4_t*>(ps + (wm * 128 + t * 32 + l32) * LDK + kk);
    }
  };
  auto compute = [&](int st) {
    u32x4_t fa[2][4], fb[2][4];
    frags(st, 0, fa[0], fb[0]);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      if (ks + 1 < BK / 16) frags(st, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
          acc[tj][ti] = mfma(fa[ks & 1][tj], fb[ks & 1][ti], acc[tj][ti]);
    }
  };

  {
    // Loads past the last slab re-read the last slab (clamped index) instead of
    // being skipped: uniform code lets the compiler wait for exactly the slab
    // it stages (a partial vmcnt) rather than for every load in flight.
    u32x4_t rg[DEPTH][2 * CH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) issue(d < nk ? d : nk - 1, rg[d]);
    stage_in(rg[0], 0);
    issue(DEPTH < nk ? DEPTH : nk - 1, rg[0]);
    __syncthreads();
    for (int kt0 = 0; kt0 < nk; kt0 += DEPTH) {
#pragma unroll
      for (int u = 0; u < DEPTH; ++u) {
        const int kt = kt0 + u;
        compute(u & 1);
        stage_in(rg[(u + 1) % DEPTH], (u + 1) & 1);  // (past the end: unused)
        const int nxt = kt + 1 + DEPTH;
        issue(nxt < nk ? nxt : nk - 1, rg[(u + 1) % DEPTH]);
        __syncthreads();
      }
    }
  }

  // Epilogue. Lane holds C[i][j..j+3], i = row0 + l32, j = col0 + 8q + 4hi.
  // The R operand (A or X) of all 64 groups is loaded before any store: a
  // load issued after stores would wait for them (in-order vmcnt).
  uint16_t* const img = lds;  // the stage buffers are free now
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
        float x = bf16_to_f32(half16(rv[e >> 1], e & 1));
        if constexpr (MODE == kApply) {
          if constexpr (SCALED) x = round_bf16(x * sc);
          h[e] = f32_to_bf16(fmaf(g.beta, x, round_bf16(v[e])));
        } else {
          h[e] = f32_to_bf16(fmaf(g.beta, x, g.alpha * v[e]));
        }
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
      const u32x4_t val = *reinterpret_cast<const u32x4_t*>(img + r * LDI + c8);
      *reinterpret_cast<u32x4_t*>(Dt + (int64_t)(bj * BT + pass * IMGR + r) * ldd + bi * BT + c8) =
          val;
    }
    __syncthreads();
  }
}

template <int MODE, bool SCALED>
__global__ __launch_bounds__(NT, 1) void ns_nt_kernel(NtArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_ELEMS];
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
    nt_item<MODE, SCALED>(g, lds, tile, bi, bj);
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

template <int MODE, bool SCALED>
void launch(const NtArgs& a, int64_t items, hipStream_t s) {
  const int64_t per_xcd = (items + 7) / 8;
  const int64_t wgs_per_xcd = std::max<int64_t>(1, std::min<int64_t>(num_cus() / 8, per_xcd));
  hipLaunchKernelGGL((ns_nt_kernel<MODE, SCALED>), dim3((unsigned)(8 * wgs_per_xcd)), dim3(NT), 0,
                     s, a);
}

}  // namespace

bool ns5_nt_supported(int mp, int np) { return mp % BT == 0 && np % BT == 0; }

// One sub-batch of `cnt` tiles, `steps` iterations, ping-ponging X between
// (x, xt) and (y, yt); A and B live in the workspace.
void ns5_nt_run(uint16_t* x, uint16_t* xt, uint16_t* y, uint16_t* yt, const float* inv,
                int64_t cnt, int mp, int np, int steps, float a, float b, float c, uint16_t* wsA,
                uint16_t* wsB, hipStream_t s) {
  const int64_t sq = (int64_t)mp * mp, rect = (int64_t)mp * np;
  const int nb = mp / BT;
  const int64_t gram_items = cnt * (nb * (nb + 1) / 2);
  const int64_t apply_items = cnt * nb * (np / BT);
  uint16_t* cur = x;
  uint16_t* curT = xt;
  uint16_t* nxt = y;
  uint16_t* nxtT = yt;
  for (int it = 0; it < steps; ++it) {
    const bool first = it == 0, last = it == steps - 1;
    NtArgs ga{cur, rect, np, cur, rect, np, nullptr, 0, 0, wsA, sq, mp, nullptr, 0, 0,
              first ? inv : nullptr, mp, mp, np, cnt, 1.0f, 0.0f};
    if (first) launch<kGramA, true>(ga, gram_items, s);
    else launch<kGramA, false>(ga, gram_items, s);
    NtArgs gb{wsA, sq, mp, wsA, sq, mp, wsA, sq, mp, wsB, sq, mp, nullptr, 0, 0,
              nullptr, mp, mp, mp, cnt, c, b};
    launch<kGramB, false>(gb, gram_items, s);
    NtArgs ap{wsB, sq, mp, curT, rect, mp, cur, rect, np, nxt, rect, np, last ? nullptr : nxtT,
              rect, mp, first ? inv : nullptr, mp, np, mp, cnt, 1.0f, a};
    if (first) launch<kApply, true>(ap, apply_items, s);
    else launch<kApply, false>(ap, apply_items, s);
    std::swap(cur, nxt);
    std::swap(curT, nxtT);
  }
}
