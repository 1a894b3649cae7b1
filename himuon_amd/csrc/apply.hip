// Weight decay + learning-rate application after the captured step, for
// every parameter in one launch per (parameter dtype, update dtype) pair
// (himuon.py:215-228 `_apply_pending_updates`):
//
//     p.mul_(1 - lr * wd)          p1 = round_p(float(p) * s)
//     p.add_(update, alpha=-lr)    p  = round_p(fma(alpha, round_p(u), p1))
//
// with s = float(1 - lr * wd) and alpha = float(-lr) per param group, the
// values torch's two elementwise kernels compute in fp32 opmath: the in-place
// add first rounds `other` to the parameter's dtype (a no-op for fp32
// parameters), then evaluates `self + alpha * other` as one fused
// multiply-add (verified bit for bit against torch on the GPU). For fp16
// parameters with an fp32 update torch's mixed-dtype add rounds that
// multiply-add once from the exact value instead of through fp32
// (fma_f16_once, measured over 1 M elements); other pairs go through fp32.
// With wd == 0 the first line is the identity, as the reference's skipped mul_.
//
// HBM-bound: read p, read u, write p (8 B per element for bf16 params and
// fp32 updates, against 12 B for the two separate torch passes). Work is cut
// into chunks of 8192 elements per parameter; a persistent grid walks the
// chunks, each thread issuing the loads of its four 8-element vectors before
// using them.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kVec = 4;       // 8-element vectors per thread per chunk
constexpr int kChunk = kThreads * kVec * 8;  // 8192 elements

struct ApplyScalars {
  float s[HIMUON_APPLY_MAX_GROUPS];
  float alpha[HIMUON_APPLY_MAX_GROUPS];
};

// (s_g, alpha_g) pairs into the device table the fused untile reads. The
// values travel as launch arguments, so the write is stream-ordered behind
// earlier work (a graph replay still reading the table) and needs no host
// buffer that outlives the call.
__global__ __launch_bounds__(64) void write_scale_alpha_kernel(float* __restrict__ out, ApplyScalars sc,
                                                               int n_groups) {
  const int g = threadIdx.x;
  if (g < n_groups) {
    out[2 * g] = sc.s[g];
    out[2 * g + 1] = sc.alpha[g];
  }
}

// Descriptor owning chunk q: the last d with descs[d].chunk0 <= q.
HM_DEV int find_desc(const HimuonApplyDesc* __restrict__ d, int n, int64_t q) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (d[mid].chunk0 <= q) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// p1 + alpha * round_p(u), stored in the parameter dtype PD (see above).
template <int PD, int UD>
HM_DEV float add_update(float alpha, float u, float p1) {
  if constexpr (PD == HIMUON_DTYPE_F16 && UD == HIMUON_DTYPE_F32)
    return fma_f16_once(alpha, round_to<PD>(u), p1);
  else
    return __builtin_fmaf(alpha, round_to<PD>(u), p1);
}

template <int PD, int UD>
__global__ __launch_bounds__(kThreads) void apply_kernel(const HimuonApplyDesc* __restrict__ descs,
                                                         int n_descs, int64_t n_chunks,
                                                         ApplyScalars sc) {
#pragma clang fp contract(off)
  for (int64_t q = blockIdx.x; q < n_chunks; q += gridDim.x) {
    const HimuonApplyDesc& D = descs[find_desc(descs, n_descs, q)];
    const float s = sc.s[D.group], alpha = sc.alpha[D.group];
    const int64_t base = (q - D.chunk0) * kChunk;
    float p[kVec][8], u[kVec][8];
    // Every load of the chunk is issued before any is used.
#pragma unroll
    for (int h = 0; h < kVec; ++h) {
      const int64_t e0 = base + (int64_t)(h * kThreads + threadIdx.x) * 8;
      if (e0 + 8 <= D.numel) {
        load8<PD>(D.param, e0, p[h]);
        load8<UD>(D.update, e0, u[h]);
      }
    }
#pragma unroll
    for (int h = 0; h < kVec; ++h) {
      const int64_t e0 = base + (int64_t)(h * kThreads + threadIdx.x) * 8;
      if (e0 >= D.numel) continue;
      if (e0 + 8 <= D.numel) {
#pragma unroll
        for (int e = 0; e < 8; ++e) p[h][e] = add_update<PD, UD>(alpha, u[h][e], round_to<PD>(p[h][e] * s));
        store8<PD>(D.param, e0, p[h]);
      } else {
        for (int64_t e = e0; e < D.numel; ++e) {
          const float p1 = round_to<PD>(load_elem<PD>(D.param, e) * s);
          store_elem<PD>(D.param, e, add_update<PD, UD>(alpha, load_elem<UD>(D.update, e), p1));
        }
      }
    }
  }
}

template <int PD>
int launch_pd(int ud, const HimuonApplyDesc* d, int n, int64_t n_chunks, const ApplyScalars& sc,
              hipStream_t s) {
  int dev = 0, ncu = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  const dim3 grid((unsigned)std::min<int64_t>(n_chunks, (int64_t)8 * std::max(ncu, 1))), block(kThreads);
  switch (ud) {
    case HIMUON_DTYPE_F32: hipLaunchKernelGGL((apply_kernel<PD, HIMUON_DTYPE_F32>), grid, block, 0, s, d, n, n_chunks, sc); break;
    case HIMUON_DTYPE_BF16: hipLaunchKernelGGL((apply_kernel<PD, HIMUON_DTYPE_BF16>), grid, block, 0, s, d, n, n_chunks, sc); break;
    case HIMUON_DTYPE_F16: hipLaunchKernelGGL((apply_kernel<PD, HIMUON_DTYPE_F16>), grid, block, 0, s, d, n, n_chunks, sc); break;
    default: return HIMUON_EINVAL;
  }
  return (int)hipGetLastError();
}

}  // namespace

extern "C" int64_t himuon_apply_chunk_elems(void) { return kChunk; }

extern "C" int himuon_write_scale_alpha(float* scale_alpha_dev, const float* scale_by_group,
                                        const float* alpha_by_group, int n_groups, void* stream) {
  if (!scale_alpha_dev || !scale_by_group || !alpha_by_group || n_groups <= 0 ||
      n_groups > HIMUON_APPLY_MAX_GROUPS)
    return HIMUON_EINVAL;
  ApplyScalars sc{};
  for (int g = 0; g < n_groups; ++g) {
    sc.s[g] = scale_by_group[g];
    sc.alpha[g] = alpha_by_group[g];
  }
  static_assert(HIMUON_APPLY_MAX_GROUPS <= 64, "one thread per group");
  hipLaunchKernelGGL(write_scale_alpha_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                     scale_alpha_dev, sc, n_groups);
  return (int)hipGetLastError();
}

extern "C" int himuon_apply_updates(const HimuonApplyDesc* descs_dev, int n_descs, int64_t n_chunks,
                                    int param_dtype, int update_dtype, const float* scale_by_group,
                                    const float* alpha_by_group, int n_groups, void* stream) {
  if (!descs_dev || n_descs <= 0 || n_chunks < 0 || !scale_by_group || !alpha_by_group ||
      n_groups <= 0 || n_groups > HIMUON_APPLY_MAX_GROUPS)
    return HIMUON_EINVAL;
  if (n_chunks == 0) return 0;
  ApplyScalars sc{};
  for (int g = 0; g < n_groups; ++g) {
    sc.s[g] = scale_by_group[g];
    sc.alpha[g] = alpha_by_group[g];
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (param_dtype) {
    case HIMUON_DTYPE_F32: return launch_pd<HIMUON_DTYPE_F32>(update_dtype, descs_dev, n_descs, n_chunks, sc, s);
    case HIMUON_DTYPE_BF16: return launch_pd<HIMUON_DTYPE_BF16>(update_dtype, descs_dev, n_descs, n_chunks, sc, s);
    case HIMUON_DTYPE_F16: return launch_pd<HIMUON_DTYPE_F16>(update_dtype, descs_dev, n_descs, n_chunks, sc, s);
    default: return HIMUON_EINVAL;
  }
}
