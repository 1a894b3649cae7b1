// AdamW fallback for the parameters of the non-Muon groups (embeddings,
// norms, lm_head), inside the captured step: himuon.py:359-372
// (`_compute_adamw_step`) and 878-888 (`_step_adamw`). The reference runs it
// as a chain of torch ops per parameter:
//
//     step.add_(1)
//     m.lerp_(g, 1 - b1);  v.lerp_(g.square(), 1 - b2)
//     bc1 = 1 - b1 ** step;  bc2 = 1 - b2 ** step
//     update = (m / bc1) / (v.sqrt() / bc2 ** 0.5 + eps)
//
// Every op stores its result in the moment dtype T (the grad dtype), so the
// kernel rounds at the same points (rd = round to T; fp32 arithmetic):
//
//     m   = rd(lerp(m, g, w1))           lerp(a, b, w) = fma(w, b - a, a) for |w| < 0.5,
//     v   = rd(lerp(v, rd(g * g), w2))                   fma(-(b - a), 1 - w, b) otherwise
//     u   = rd(rd(m / bc1) / rd(rd(rd(sqrt(v)) / sbc2) + eps))
//
// with w = float(1 - beta) formed in double as Python does, bc1 = 1 - powf(b1,
// step), sbc2 = sqrtf(1 - powf(b2, step)) in fp32; for bf16/fp16 moments bc1
// and sbc2 enter the divisions rounded to T (torch's GPU kernels cast a 0-dim
// fp32 operand to the common dtype before the op; the Python-float eps goes to
// fp32 directly). torch's GPU kernels were checked on the MI355X to evaluate
// lerp as that fma, division and sqrt correctly rounded, and `beta ** step`
// with the device library's powf (not correctly rounded), which is what powf
// below calls.
//
// Two launches: a per-parameter prep (step += 1, bias corrections into a
// small device table), then one persistent multi-tensor elementwise pass:
// read g, m, v and write m, v, u, 24 B per fp32 element, against about 76 B
// for the reference's separate ops. The WD/LR application of the update stays
// outside the graph, as in the reference.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kVec = 2;                      // 8-element vectors per thread per chunk
constexpr int kChunk = kThreads * kVec * 8;  // 4096 elements

struct AdamwScalars {
  float w1[HIMUON_ADAMW_MAX_GROUPS];   // float(1 - beta1)
  float w2[HIMUON_ADAMW_MAX_GROUPS];   // float(1 - beta2)
  float b1[HIMUON_ADAMW_MAX_GROUPS];   // float(beta1)
  float b2[HIMUON_ADAMW_MAX_GROUPS];   // float(beta2)
  float eps[HIMUON_ADAMW_MAX_GROUPS];  // float(eps)
};

HM_DEV int find_desc(const HimuonAdamwDesc* __restrict__ d, int n, int64_t q) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (d[mid].chunk0 <= q) lo = mid; else hi = mid - 1;
  }
  return lo;
}

HM_DEV float lerp32(float a, float b, float w) {
  const float d = b - a;
  return fabsf(w) < 0.5f ? __builtin_fmaf(w, d, a) : __builtin_fmaf(-d, 1.0f - w, b);
}

// bias[2 d] = bc1, bias[2 d + 1] = sqrt(bc2) after the step increment.
__global__ __launch_bounds__(kThreads) void adamw_prep_kernel(const HimuonAdamwDesc* __restrict__ descs,
                                                              int n_descs, AdamwScalars sc,
                                                              float* __restrict__ bias) {
#pragma clang fp contract(off)
  const int d = blockIdx.x * kThreads + threadIdx.x;
  if (d >= n_descs) return;
  const HimuonAdamwDesc& D = descs[d];
  const float s = *D.step + 1.0f;
  *D.step = s;
  const float bc1 = 1.0f - powf(sc.b1[D.group], s);
  const float bc2 = 1.0f - powf(sc.b2[D.group], s);
  bias[2 * d] = bc1;
  bias[2 * d + 1] = sqrtf(bc2);
}

template <int T>
HM_DEV void adamw_elem(float g, float& m, float& v, float& u, float w1, float w2, float bc1, float sbc2,
                       float eps) {
#pragma clang fp contract(off)
  m = round_to<T>(lerp32(m, g, w1));
  v = round_to<T>(lerp32(v, round_to<T>(g * g), w2));
  const float t1 = round_to<T>(m / bc1);
  const float t2 = round_to<T>(sqrtf(v));
  const float t3 = round_to<T>(round_to<T>(t2 / sbc2) + eps);
  u = round_to<T>(t1 / t3);
}

template <int T>
__global__ __launch_bounds__(kThreads) void adamw_kernel(const HimuonAdamwDesc* __restrict__ descs,
                                                         int n_descs, int64_t n_chunks, AdamwScalars sc,
                                                         const float* __restrict__ bias) {
  for (int64_t q = blockIdx.x; q < n_chunks; q += gridDim.x) {
    const int di = find_desc(descs, n_descs, q);
    const HimuonAdamwDesc& D = descs[di];
    const float w1 = sc.w1[D.group], w2 = sc.w2[D.group], eps = sc.eps[D.group];
    const float bc1 = round_to<T>(bias[2 * di]), sbc2 = round_to<T>(bias[2 * di + 1]);
    const int64_t base = (q - D.chunk0) * kChunk;
    float g[kVec][8], m[kVec][8], v[kVec][8];
#pragma unroll
    for (int h = 0; h < kVec; ++h) {
      const int64_t e0 = base + (int64_t)(h * kThreads + threadIdx.x) * 8;
      if (e0 + 8 <= D.numel) {
        load8<T>(D.grad, e0, g[h]);
        load8<T>(D.moment1, e0, m[h]);
        load8<T>(D.moment2, e0, v[h]);
      }
    }
#pragma unroll
    for (int h = 0; h < kVec; ++h) {
      const int64_t e0 = base + (int64_t)(h * kThreads + threadIdx.x) * 8;
      if (e0 >= D.numel) continue;
      if (e0 + 8 <= D.numel) {
        float u[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) adamw_elem<T>(g[h][e], m[h][e], v[h][e], u[e], w1, w2, bc1, sbc2, eps);
        store8<T>(D.moment1, e0, m[h]);
        store8<T>(D.moment2, e0, v[h]);
        store8<T>(D.update, e0, u);
      } else {
        for (int64_t e = e0; e < D.numel; ++e) {
          float mm = load_elem<T>(D.moment1, e), vv = load_elem<T>(D.moment2, e), uu;
          adamw_elem<T>(load_elem<T>(D.grad, e), mm, vv, uu, w1, w2, bc1, sbc2, eps);
          store_elem<T>(D.moment1, e, mm);
          store_elem<T>(D.moment2, e, vv);
          store_elem<T>(D.update, e, uu);
        }
      }
    }
  }
}

}  // namespace

extern "C" int64_t himuon_adamw_chunk_elems(void) { return kChunk; }

extern "C" int himuon_adamw_step(const HimuonAdamwDesc* descs_dev, int n_descs, int64_t n_chunks, int dtype,
                                 const double* beta1_by_group, const double* beta2_by_group,
                                 const double* eps_by_group, int n_groups, float* bias_dev, void* stream) {
  if (!descs_dev || n_descs <= 0 || n_chunks < 0 || !beta1_by_group || !beta2_by_group || !eps_by_group ||
      n_groups <= 0 || n_groups > HIMUON_ADAMW_MAX_GROUPS || !bias_dev)
    return HIMUON_EINVAL;
  if (dtype != HIMUON_DTYPE_F32 && dtype != HIMUON_DTYPE_BF16 && dtype != HIMUON_DTYPE_F16)
    return HIMUON_EINVAL;
  AdamwScalars sc{};
  for (int g = 0; g < n_groups; ++g) {
    sc.w1[g] = (float)(1.0 - beta1_by_group[g]);
    sc.w2[g] = (float)(1.0 - beta2_by_group[g]);
    sc.b1[g] = (float)beta1_by_group[g];
    sc.b2[g] = (float)beta2_by_group[g];
    sc.eps[g] = (float)eps_by_group[g];
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(adamw_prep_kernel, dim3((unsigned)((n_descs + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     s, descs_dev, n_descs, sc, bias_dev);
  if (n_chunks == 0) return (int)hipGetLastError();
  int dev = 0, ncu = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  const dim3 grid((unsigned)std::min<int64_t>(n_chunks, (int64_t)8 * std::max(ncu, 1))), block(kThreads);
  switch (dtype) {
    case HIMUON_DTYPE_F32:
      hipLaunchKernelGGL((adamw_kernel<HIMUON_DTYPE_F32>), grid, block, 0, s, descs_dev, n_descs, n_chunks, sc, bias_dev);
      break;
    case HIMUON_DTYPE_BF16:
      hipLaunchKernelGGL((adamw_kernel<HIMUON_DTYPE_BF16>), grid, block, 0, s, descs_dev, n_descs, n_chunks, sc, bias_dev);
      break;
    default:
      hipLaunchKernelGGL((adamw_kernel<HIMUON_DTYPE_F16>), grid, block, 0, s, descs_dev, n_descs, n_chunks, sc, bias_dev);
      break;
  }
  return (int)hipGetLastError();
}
