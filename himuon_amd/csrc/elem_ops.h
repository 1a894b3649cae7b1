// Per-element arithmetic of the step shared by the tile kernels and the
// fused LDS-resident step kernel: the momentum update (the gather) and the
// WD/LR application of the update to a parameter (the fused untile).
#pragma once

#include "common.h"

// Momentum for one element (himuon.py:354-356); returns the NS input and
// writes the new momentum value to *m. Results are rounded to the tensor
// dtype where torch stores them: buf.mul_(mu) and .add_(g) each store (two
// roundings, no contraction); g.add(buf, alpha=mu) is one fp32 fused
// multiply-add stored once, as torch evaluates `self + alpha * other`.
template <int DT>
HM_DEV float momentum_elem(float g, float* m, float mu, bool nesterov, bool has_mom) {
  // (__fmul_rn/__fadd_rn would still be contracted into an FMA; plain
  // operators under contract(off) are not.)
#pragma clang fp contract(off)
  if (!has_mom) return g;
  const float prod = round_to<DT>(mu * *m);
  const float mb = round_to<DT>(prod + g);
  *m = mb;
  if (!nesterov) return mb;
  return round_to<DT>(__builtin_fmaf(mu, mb, g));
}

// The WD/LR step of the fused untile (himuon_untile_apply, and the fused NS
// kernel's last iteration) on parameter values p and their updates y:
//     p = rd(fma(alpha, rd(y), rd(p s)))
// wdlr8: 8 values p already loaded as fp32 (rounded to DT by the store that
// follows); wdlr_elems: the first `valid` elements at base + o, one at a time.
template <int DT>
HM_DEV void wdlr8(float (&p)[8], const float (&y)[8], float s, float alpha) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = __builtin_fmaf(alpha, round_to<DT>(y[e]), round_to<DT>(p[e] * s));
}
template <int DT>
HM_DEV void wdlr_elems(void* base, int64_t o, const float (&y)[8], int valid, float s, float alpha) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 8; ++e) {  // (static indices: y stays in registers)
    if (e < valid) {
      const float p1 = round_to<DT>(load_elem<DT>(base, o + e) * s);
      store_elem<DT>(base, o + e, __builtin_fmaf(alpha, round_to<DT>(y[e]), p1));
    }
  }
}

// Untile store of 8 consecutive update values y (fp32, already scaled by the
// parameter's upd_scale) at element offset o of descriptor P's `update`;
// `full`: all 8 in range and 16-byte aligned, else the first `valid` one at a
// time. APPLY: `update` is the parameter itself (ld_upd its row stride) and
// the weight decay and learning rate of its group are applied in place
// instead of storing the update (himuon_untile_apply):
//     p = rd(fma(alpha_g, rd(u), rd(p * s_g))),  u = upd_scale * NS (fp32)
// rd the rounding to DT; sa holds (s_g, alpha_g) per group, in device memory.
template <bool APPLY, int DT>
HM_DEV void put8(const HimuonParamDesc& P, int64_t o, const float (&y)[8], bool full, int valid,
                 const float* __restrict__ sa) {
#pragma clang fp contract(off)
  if constexpr (APPLY) {
    const float s = sa[2 * P.group], alpha = sa[2 * P.group + 1];
    if (full) {
      float p[8];
      load8<DT>(P.update, o, p);
      wdlr8<DT>(p, y, s, alpha);
      store8<DT>(P.update, o, p);
    } else {
      wdlr_elems<DT>(P.update, o, y, valid, s, alpha);
    }
  } else {
    if (full) {
      store8<DT>(P.update, o, y);
    } else {
      for (int e = 0; e < valid; ++e) store_elem<DT>(P.update, o + e, y[e]);
    }
  }
}

