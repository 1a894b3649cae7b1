/*
 * himuon_hip.h — C ABI of libhimuon_hip.so, the MI355X (gfx950) kernels behind
 * the HiMuon optimizer step.
 *
 * The library replaces the GPU bodies of the reference optimizer's step
 * (tang0389/himuon, src/himuon/optimizers/himuon.py). Host code (Python/ctypes
 * in himuon_amd/_native.py) owns every buffer; nothing here allocates device
 * memory, synchronises the device or keeps mutable global state, so every entry
 * point may be recorded into a hipGraph. All launches go to the caller's
 * stream. All entry points return 0 on success, a positive hipError_t from the
 * launch, or a negative HIMUON_E* code for an argument error found on the host
 * before anything was launched.
 *
 * Data layout shared by the entry points
 * --------------------------------------
 *  Bucket geometry: every parameter of a bucket is cut into tile_h x tile_w
 *  tiles (zero padded at the bottom/right edge of the parameter). A tile is
 *  "transposed" when tile_h > tile_w: the Newton-Schulz (NS) operand is then
 *  the tile's transpose, so NS always sees an m x n matrix with m <= n,
 *  m = min(tile_h, tile_w), n = max(tile_h, tile_w).
 *
 *  NS tile buffer: bf16, shape (n_tiles, mp, np) row-major, mp >= m and
 *  np >= n multiples of HIMUON_NS_ALIGN. NS tile t holds the tile at
 *  bucket tile index t in its top-left m x n corner and zeros elsewhere
 *  (zero rows/columns stay exactly zero through NS).
 *
 *  Tile numbering: parameter p owns tiles [tile0_p, tile0_p + R_p*C_p); tile
 *  (r, c) of the parameter's R_p x C_p tile grid is tile0_p + r*C_p + c
 *  (row-major), the concat-buffer order of himuon.py:677-719.
 */
#ifndef HIMUON_HIP_H
#define HIMUON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HIMUON_ABI_VERSION 5

/* Element type codes for gradients / momentum / updates. */
#define HIMUON_DTYPE_F32 0
#define HIMUON_DTYPE_BF16 1
#define HIMUON_DTYPE_F16 2
/* fp8 e5m2 (OCP: 5 exponent bits, bias 15): operands of the typed stage
 * products only (himuon_*_typed). */
#define HIMUON_DTYPE_E5M2 3

/* NS tile buffer dimensions (mp, np) must be multiples of this. */
#define HIMUON_NS_ALIGN 128

/* Host-side argument errors (negative return codes). */
#define HIMUON_EINVAL (-22)
#define HIMUON_ENOSPC (-28)

/*
 * One parameter of a bucket. An array of these lives in device memory (built
 * once per plan by the host) and is read by the gather and untile kernels.
 * 96 bytes, 8-byte aligned; field order is part of the ABI. Parameters of one
 * bucket may come from different param groups, so the per-group momentum
 * settings travel with each parameter.
 */
typedef struct HimuonParamDesc {
  const void* grad;   /* (h, w) gradient, row stride ld_grad elements          */
  void* momentum;     /* (h, w) momentum buffer, row stride ld_mom; may be NULL */
  void* update;       /* (h, w) update output, row stride ld_upd                */
  int64_t h, w;
  int64_t ld_grad, ld_mom, ld_upd;
  int64_t tile0;      /* first NS tile index of this parameter                  */
  int32_t R, C;       /* tile grid: ceil(h / tile_h) x ceil(w / tile_w)         */
  float upd_scale;    /* update = upd_scale * NS output (lr adjustment)          */
  float mu;           /* momentum coefficient                                    */
  int32_t nesterov;   /* nonzero: Nesterov momentum                              */
  int32_t group;      /* param group index (read by himuon_untile_apply only)    */
} HimuonParamDesc;

/* Library ABI version (HIMUON_ABI_VERSION it was built with). */
int himuon_abi_version(void);

/* Human-readable text for any return code of this library. */
const char* himuon_error_string(int code);

/* Number of fp32 sum-of-squares partials himuon_momentum_gather writes per NS
 * tile for this geometry (the row length of its `partials` output). */
int himuon_gather_partials_per_tile(int tile_h, int tile_w, int mp, int np);

/*
 * Fused Nesterov momentum + tile gather + per-tile sum of squares.
 * Replaces the per-parameter pre-NS loop of himuon.py:696-719
 * (_compute_momentum himuon.py:350-357, F.pad + permute-copy into the concat
 * buffer) and the bf16 cast of the NS prologue (himuon.py:239, 274).
 *
 * For every element of every parameter (grad g, momentum buf, both in
 * `dtype`; mu and nesterov from the parameter's descriptor):
 *     buf <- rd(rd(mu * buf) + g)                      (in place)
 *     e   <- nesterov ? rd(fma(mu, buf, g)) : buf
 * (fp32 arithmetic; rd = round to `dtype`; the buf update rounds its product
 * and sum separately, e is one fused multiply-add, as torch's in-place mul_,
 * add_ and add(alpha=) evaluate them). If momentum is NULL, e = g and
 * nothing is written back. bf16(e) is stored at its NS tile position in
 * tiles_bf16 (n_tiles, mp, np); padding is written as zero. partials[t * P +
 * q] receives the fp32 sum of squares of the bf16 values of the q-th part of
 * NS tile t, P = himuon_gather_partials_per_tile(...): slabs of r NS rows
 * when tile_h <= tile_w, r the largest power of two with r * np <= 16384,
 * clamped to [32, mp] (P = mp / r); 64x64 blocks (P = mp/64 * np/64) for
 * tall tiles.
 */
int himuon_momentum_gather(const HimuonParamDesc* params_dev, int n_params,
                           int64_t n_tiles, int tile_h, int tile_w, int mp,
                           int np, int dtype, uint16_t* tiles_bf16,
                           float* partials, void* stream);

/*
 * Per-tile normaliser: inv[t] = 1 / (sqrt(sum_q partials[t*P+q]) + eps).
 * The reciprocal of the divisor of himuon.py:242 / ns5_smem.py:84-86
 * (Frobenius norm of the bf16 tile, fp32).
 */
int himuon_tile_scale(const float* partials, int partials_per_tile,
                      int64_t n_tiles, float eps, float* inv, void* stream);

/* Workspace bytes himuon_ns5 needs for a given sub-batch size: the bf16 A and
 * B intermediates (mp x mp each) of `sub_batch` tiles. */
size_t himuon_ns5_workspace_bytes(int64_t sub_batch, int mp, int np);

/*
 * Batched quintic Newton-Schulz on n_tiles NS tiles.
 * Replaces HiMuon.newton_schulz / _newton_schulz_3kernel / ns5_smem
 * (himuon.py:232-284; triton_kernels/XXT.py:13-75, ba_plus_cAA.py:13-89,
 * fused_bmm_add.py:13-96, ns5_smem.py:46-104).
 *
 *   X0 = bf16(x * inv[t])                 (x = the gathered bf16 tile)
 *   repeat `steps` times:
 *     A = bf16(X X^T)                       fp32 accumulation
 *     B = bf16(c * (A A^T) + b * A)          fp32 accumulation / epilogue
 *     X = bf16(bf16(B X) + a * X)
 *
 * x, y: (n_tiles, mp, np) bf16; X ping-pongs between them, so the result is
 * in x when `steps` is even and in y when it is odd (the other buffer's
 * contents are unspecified afterwards; x and y must not alias). X0 is formed
 * by the first iteration's kernels as they read x, not by a separate pass.
 * Tiles with mp == 128 and np in {128, 256, 512} run all iterations
 * of a tile inside one workgroup's LDS; 512 x 512 tiles run the first
 * product on a persistent 256x256-block kernel and the other two fused
 * (himuon_ba_bmm_add's kernel); other tiles whose mp and np are multiples of
 * 256 run the three products on persistent 256x256-block kernels; other
 * geometries on 128x128-block kernels. Tiles are processed in sub-batches of `sub_batch`;
 * the workspace must hold himuon_ns5_workspace_bytes(sub_batch, mp, np)
 * bytes whenever steps > 0.
 */
int himuon_ns5(uint16_t* x, uint16_t* y, const float* inv, int64_t n_tiles,
               int mp, int np, int steps, float a, float b, float c,
               void* workspace, size_t workspace_bytes, int64_t sub_batch,
               void* stream);

/*
 * himuon_ns5 with option flags (himuon_ns5 is flags == 0):
 *  - HIMUON_NS_ROUND_ONCE: the third product of every iteration is rounded
 *    once, X = bf16(B X + a X) (fp32 B X), as the reference's 2-D path
 *    torch.addmm(X, B, X, beta=a) computes it (himuon.py:249-253; its
 *    batched 3-D path, fused_bmm_add, rounds B X first). The optimizer sets
 *    it for full-matrix parameters and 2-D newton_schulz calls.
 *  - kernel family (bits HIMUON_NS_FAMILY_MASK; no reference counterpart,
 *    for comparison tests and benchmarks): HIMUON_NS_FAMILY_AUTO picks per
 *    geometry as himuon_ns5 does; HIMUON_NS_FAMILY_BLOCK128 runs the
 *    128x128-block kernels for every geometry; HIMUON_NS_FAMILY_STREAM3 runs
 *    the three products as three streamed 256-block kernels where AUTO fuses
 *    the second and third (512 x 512 tiles). Results are identical.
 *  - HIMUON_NS_ROWS(m), m = 1 .. 64: the tiles' NS operands have only m
 *    nonzero rows (the reference's small-M shapes, e.g. 16 x 1024;
 *    himuon.py:261-284). With mp == 128, family AUTO then iterates only the
 *    first 16, 32 or 64 rows (the first that is at least m) of each tile in
 *    LDS, one workgroup per tile, for np up to 2048 (m <= 16), up to 1024
 *    (m <= 32) or 128 (m <= 64; wider 64-row tiles run the 128-row kernel,
 *    measured faster); rows from there to mp are neither read nor written (the result's rows
 *    below m are those a full computation gives; the rest of y's rows stay
 *    unspecified). Without it (0), or for other geometries, all mp rows run.
 *    The same mathematics and rounding points, in another summation order
 *    than the 128-row kernels (16 x 16 MFMA tiles).
 * Any other flag bit is an argument error.
 */
#define HIMUON_NS_FAMILY_MASK 0x0F
#define HIMUON_NS_FAMILY_AUTO 0
#define HIMUON_NS_FAMILY_BLOCK128 1
#define HIMUON_NS_FAMILY_STREAM3 2
#define HIMUON_NS_ROUND_ONCE 0x10
#define HIMUON_NS_ROWS_SHIFT 8
#define HIMUON_NS_ROWS_MASK (0x7F << HIMUON_NS_ROWS_SHIFT)
#define HIMUON_NS_ROWS(m) ((m) << HIMUON_NS_ROWS_SHIFT)
int himuon_ns5_ex(uint16_t* x, uint16_t* y, const float* inv, int64_t n_tiles,
                  int mp, int np, int steps, float a, float b, float c,
                  void* workspace, size_t workspace_bytes, int64_t sub_batch,
                  int flags, void* stream);

/*
 * The three NS products one at a time, on contiguous bf16 batches (no
 * normaliser, one product per call). They replace the reference's kernel entry
 * points XXT(A, out) (triton_kernels/XXT.py:76-104), ba_plus_cAA(A, alpha,
 * beta, out) (ba_plus_cAA.py:90-120) and fused_bmm_add(B, X, a, out)
 * (fused_bmm_add.py:98-135) with the same rounding points as himuon_ns5:
 *   himuon_xxt:         out = bf16(x x^T)            x: (batch, M, K), out: (batch, M, M)
 *   himuon_ba_plus_caa: out = bf16(alpha a a^T + beta a)   a, out: (batch, M, M)
 *   himuon_bmm_add:     out = bf16(bf16(b x) + a x)   b: (batch, M, M), x, out: (batch, M, N)
 *                       (bf16(b x + a x), one rounding, with HIMUON_NS_ROUND_ONCE:
 *                       torch.addmm(X, B, X, beta=a) of himuon.py:252-253)
 * M, N, K multiples of HIMUON_NS_ALIGN (pad with zeros: zero rows and columns
 * are exact). `flags` takes a kernel family (HIMUON_NS_FAMILY_*) and, for
 * himuon_bmm_add, HIMUON_NS_ROUND_ONCE. Outputs must not alias inputs. The
 * Gram outputs are exactly symmetric.
 */
int himuon_xxt(const uint16_t* x, uint16_t* out, int64_t batch, int M, int K,
               int flags, void* stream);
int himuon_ba_plus_caa(const uint16_t* a, uint16_t* out, int64_t batch, int M,
                       float alpha, float beta, int flags, void* stream);
/*
 * The same three products for every operand dtype the reference's kernels
 * take: tl.dot on the loaded dtype with an fp32 accumulator, the result cast to
 * the dtype of `out` (XXT.py:62-63, ba_plus_cAA.py:65-85, fused_bmm_add.py:73-88;
 * exercised with bf16, fp16, fp32 and fp8 e5m2 operands in
 * tests/integration/test_kernels.py:36-165):
 *   himuon_xxt_typed:         out = x x^T                  x: (batch, M, K)
 *   himuon_ba_plus_caa_typed: out = alpha a a^T + beta a   a: (batch, M, M)
 *   himuon_bmm_add_typed:     out = out_t(b x) + a x       b: (batch, M, M), x: (batch, M, N)
 *                             (b x rounded to the output dtype before the add)
 * in_dtype: HIMUON_DTYPE_F32, _BF16, _F16 or _E5M2 (every operand); out_dtype:
 * HIMUON_DTYPE_F32, _BF16 or _F16. bf16 and fp16 operands run the MFMAs of their
 * type, e5m2 ones the fp16 MFMA (exact widening), fp32 ones three bf16 MFMAs
 * per product (16 significant bits of each operand). M, N multiples of
 * HIMUON_NS_ALIGN, K a multiple of 64; contiguous batches; outputs must not
 * alias inputs; at most 2^31 - 8 output blocks of 128 x 128 per call.
 */
int himuon_xxt_typed(const void* x, void* out, int64_t batch, int M, int K,
                     int in_dtype, int out_dtype, void* stream);
int himuon_ba_plus_caa_typed(const void* a, void* out, int64_t batch, int M,
                             float alpha, float beta, int in_dtype,
                             int out_dtype, void* stream);
int himuon_bmm_add_typed(const void* b, const void* x, void* out,
                         int64_t batch, int M, int N, float a, int in_dtype,
                         int out_dtype, void* stream);

int himuon_bmm_add(const uint16_t* b, const uint16_t* x, uint16_t* out,
                   int64_t batch, int M, int N, float a, int flags, void* stream);

/*
 * The second and third products fused, with B kept on chip (the kernel the
 * optimizer runs for 512 x 512 tiles):
 *     out = bf16(bf16(B X) + gamma * X),  B = bf16(alpha * (A A^T) + beta * A)
 * (bf16(B X + gamma * X) with HIMUON_NS_ROUND_ONCE). No single reference
 * counterpart: it equals ba_plus_cAA (ba_plus_cAA.py:90-120) followed by
 * fused_bmm_add (fused_bmm_add.py:98-135), bit for bit. A: (batch, 512, 512)
 * bf16, exactly symmetric (an XXT output); X, out: (batch, 512, 512) bf16;
 * M == N == 512, batch < 2^29 (32-bit work-item indices; larger batches
 * return HIMUON_EINVAL); `flags` takes only HIMUON_NS_ROUND_ONCE.
 */
int himuon_ba_bmm_add(const uint16_t* a, const uint16_t* x, uint16_t* out,
                      int64_t batch, int M, int N, float alpha, float beta,
                      float gamma, int flags, void* stream);

/*
 * The whole step of a bucket whose NS tiles are 128 x 128 (tile_h <= tile_w
 * <= 128, so no tile is transposed) in one launch: for bucket tiles
 * tile_begin .. tile_begin + n_tiles - 1, himuon_momentum_gather,
 * himuon_tile_scale, himuon_ns5_ex (flags: HIMUON_NS_ROUND_ONCE only) and
 * himuon_untile_apply, with each tile held in one workgroup's LDS from the
 * momentum update to the parameter update. Replaces the per-bucket sequence
 * of himuon.py:704-719 (momentum, tiling), 232-284 (NS5) and 315-348 (untile,
 * WD/LR) for small tiles (the reference's one-kernel ns5_smem regime,
 * himuon.py:263-284). params_dev is the descriptor table of
 * himuon_momentum_gather / himuon_untile_apply (`update` = the parameter);
 * dtype (grads and momentum) and param_dtype are each HIMUON_DTYPE_F32 or
 * HIMUON_DTYPE_BF16. The momentum buffers and parameters end bit-identical to
 * those four calls; no NS tile buffer is read or written. Other geometries
 * and dtypes are an argument error.
 */
int himuon_lds_step(const HimuonParamDesc* params_dev, int n_params,
                    int64_t tile_begin, int64_t n_tiles, int tile_h,
                    int tile_w, int dtype, int param_dtype, int steps,
                    float a, float b, float c, float eps, int flags,
                    const float* scale_alpha_dev, void* stream);

/*
 * himuon_ns5_ex without a workspace argument, for callers that cannot
 * allocate (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. It allocates nothing:
 * the A/B intermediates live in a device array of HIMUON_NS_SCRATCH_BYTES
 * inside the library, one per GPU, held until the process ends, and the tiles
 * are processed in sub-batches of HIMUON_NS_SCRATCH_BYTES /
 * himuon_ns5_workspace_bytes(1, mp, np). Returns HIMUON_ENOSPC when one
 * tile's workspace exceeds HIMUON_NS_SCRATCH_BYTES (mp above 4096). Results
 * are identical to himuon_ns5_ex's. Every call on one GPU uses that GPU's
 * array: calls that overlap on one GPU (other streams or host threads) race
 * and must be serialised by the caller; nothing in the array needs to start
 * at zero. The array's device address is looked up on the first call on each
 * device (the one exception to "no mutable global state": a per-device cache
 * of that address).
 */
#define HIMUON_NS_SCRATCH_BYTES ((size_t)64 << 20)
int himuon_ns5_noalloc(uint16_t* x, uint16_t* y, const float* inv,
                       int64_t n_tiles, int mp, int np, int steps, float a,
                       float b, float c, int flags, void* stream);

/*
 * Untile/scatter: for every element of every parameter,
 *     update[row, col] = round_dtype(upd_scale * float(NS tile value))
 * reading the NS tile position of (row, col) (transposed back when
 * tile_h > tile_w). Replaces _post_ns_per_param (himuon.py:315-329; _untile
 * himuon.py:302-310), the NS output cast (himuon.py:257, 283) and the
 * in-graph `update.mul_(scale)` (himuon.py:338-341).
 */
int himuon_untile(const HimuonParamDesc* params_dev, int n_params,
                  int64_t n_tiles, int tile_h, int tile_w, int mp, int np,
                  int dtype, const uint16_t* tiles_bf16, void* stream);

/*
 * Untile and apply in place: like himuon_untile, but each descriptor's
 * `update` is the parameter itself (ld_upd its row stride, param_dtype its
 * dtype) and, instead of storing the update, the weight decay and learning
 * rate of the parameter's group (descriptor field `group`) are applied:
 *     u = upd_scale * float(NS tile value)                      (fp32)
 *     p = rd(fma(alpha[g], rd(u), rd(float(p) * scale[g])))      rd = round to param_dtype
 * with scale[g] = scale_alpha_dev[2 g], alpha[g] = scale_alpha_dev[2 g + 1]
 * read from DEVICE memory when the kernel runs, so a captured graph picks up
 * learning-rate and weight-decay changes written there before each replay.
 * The parameters end exactly as himuon_untile followed by
 * himuon_apply_updates would leave them when the update dtype is the
 * parameter dtype (the fma runs in fp32; for fp16 parameters with fp32
 * grads use the two-pass path, whose update-into-fp16 add rounds once). Replaces the untile plus the
 * outside-graph WD/LR of the Muon parameters (himuon.py:315-348, 215-228).
 */
int himuon_untile_apply(const HimuonParamDesc* params_dev, int n_params,
                        int64_t n_tiles, int tile_h, int tile_w, int mp, int np,
                        int param_dtype, const uint16_t* tiles_bf16,
                        const float* scale_alpha_dev, void* stream);

/*
 * NS5 with the untile with WD/LR fused into its last iteration: the same
 * result as himuon_ns5_ex on tiles x / y followed by himuon_untile_apply of
 * that result, for the bucket tiles tile_begin .. tile_begin + n_tiles - 1 of
 * the descriptor table (x = the bucket's tile buffer advanced to tile
 * tile_begin; the untile's tile numbering is the bucket's). The last
 * iteration's kernel applies each value to its parameter as it computes it
 * instead of writing the NS result, so x and y hold no result afterwards.
 * Supported (else HIMUON_EINVAL, nothing launched; the caller runs the two
 * calls instead) for 512 x 512 NS tiles (mp == np == 512) that are not
 * transposed (tile_h <= tile_w), family AUTO, steps >= 2 and fp32 or bf16
 * parameters; himuon_ns5_untile_apply_supported answers for a geometry.
 * Replaces newton_schulz + _post_ns_per_param + the Muon parameters'
 * outside-graph WD/LR of one chunk (himuon.py:232-284, 315-348, 215-228).
 */
int himuon_ns5_untile_apply_supported(int mp, int np, int tile_h, int tile_w, int steps, int flags,
                                      int param_dtype);
int himuon_ns5_untile_apply(uint16_t* x, uint16_t* y, const float* inv, int64_t n_tiles, int mp, int np,
                            int steps, float a, float b, float c, void* workspace, size_t workspace_bytes,
                            int64_t sub_batch, int flags, const HimuonParamDesc* params_dev, int n_params,
                            int64_t tile_begin, int tile_h, int tile_w, int param_dtype,
                            const float* scale_alpha_dev, void* stream);

/*
 * Write the table himuon_untile_apply reads: scale_alpha_dev[2 g] =
 * scale_by_group[g], scale_alpha_dev[2 g + 1] = alpha_by_group[g] for
 * g < n_groups (at most HIMUON_APPLY_MAX_GROUPS). scale_by_group and
 * alpha_by_group are HOST arrays, copied into the launch arguments, so the
 * write is a kernel on `stream`: ordered after earlier work on it (a graph
 * replay that still reads the table) and asynchronous to the host, like the
 * Python-float lr and wd the reference's outside-graph WD/LR uses
 * (himuon.py:215-228). Call it outside any captured graph, before each replay.
 */
int himuon_write_scale_alpha(float* scale_alpha_dev, const float* scale_by_group,
                             const float* alpha_by_group, int n_groups, void* stream);

/*
 * Weight decay + learning-rate application, outside the captured graph
 * (replaces _apply_pending_updates, himuon.py:215-228, and the eager
 * _apply_wd_and_update, himuon.py:333-348). One descriptor per parameter, in
 * device memory, built once per capture; each parameter's elements are cut
 * into chunks of himuon_apply_chunk_elems() and descriptor d owns chunks
 * [chunk0_d, chunk0_d + ceil(numel_d / chunk)) of the launch. param and
 * update must be contiguous and 16-byte aligned. For every element:
 *     p1 = round_p(float(p) * scale[group]);          p.mul_(1 - lr*wd)
 *     p  = round_p(fma(alpha[group], round_p(u), p1)) p.add_(u, alpha=-lr)
 * with the fma in fp32, except for fp16 parameters with an fp32 update,
 * where (as torch's mixed-dtype add does) p1 + alpha * round_p(u) is rounded
 * to fp16 once from its exact value.
 * scale_by_group / alpha_by_group are HOST arrays of n_groups floats (copied
 * into the launch), so lr and wd may change every step without re-recording.
 * One launch covers the descriptors of one (param dtype, update dtype) pair.
 */
#define HIMUON_APPLY_MAX_GROUPS 32

typedef struct HimuonApplyDesc {
  void* param;         /* contiguous parameter                          */
  const void* update;  /* contiguous update, same number of elements    */
  int64_t numel;
  int64_t chunk0;      /* first chunk of this parameter in the launch    */
  int32_t group;       /* index into scale_by_group / alpha_by_group     */
  int32_t reserved;
} HimuonApplyDesc;

int64_t himuon_apply_chunk_elems(void);

int himuon_apply_updates(const HimuonApplyDesc* descs_dev, int n_descs,
                         int64_t n_chunks, int param_dtype, int update_dtype,
                         const float* scale_by_group,
                         const float* alpha_by_group, int n_groups,
                         void* stream);

/*
 * AdamW fallback step for the parameters of the non-Muon groups, inside the
 * captured step (replaces _compute_adamw_step, himuon.py:359-372, called from
 * _step_adamw, himuon.py:878-888). One descriptor per parameter, in device
 * memory; grad, moment1, moment2 and update are contiguous, 16-byte aligned
 * and of one dtype (`dtype`, the grad dtype); step points at the parameter's
 * fp32 step counter. Descriptor d owns chunks [chunk0_d, chunk0_d +
 * ceil(numel_d / himuon_adamw_chunk_elems())). For each parameter:
 *     step += 1; bc1 = 1 - powf(b1, step); sbc2 = sqrtf(1 - powf(b2, step))
 * and for each element (rd = round to dtype, fp32 arithmetic):
 *     m = rd(lerp(m, g, 1 - b1)); v = rd(lerp(v, rd(g*g), 1 - b2))
 *     update = rd(rd(m / rd(bc1)) / rd(rd(rd(sqrt(v)) / rd(sbc2)) + eps))
 * lerp as torch evaluates it (one fma). beta1/beta2/eps are HOST arrays of
 * n_groups doubles (the Python floats; 1 - beta is formed in double and then
 * rounded, as the reference's lerp weight is). bias_dev is device scratch of
 * 2 * n_descs floats that receives (bc1, sbc2) per descriptor.
 */
#define HIMUON_ADAMW_MAX_GROUPS 32

typedef struct HimuonAdamwDesc {
  const void* grad;   /* contiguous gradient                                */
  void* moment1;      /* contiguous first moment (exp_avg), updated in place */
  void* moment2;      /* contiguous second moment, updated in place          */
  void* update;       /* contiguous output                                   */
  float* step;        /* fp32 step counter of this parameter (device)        */
  int64_t numel;
  int64_t chunk0;     /* first chunk of this parameter in the launch          */
  int32_t group;      /* index into the per-group hyper-parameter arrays      */
  int32_t reserved;
} HimuonAdamwDesc;

int64_t himuon_adamw_chunk_elems(void);

int himuon_adamw_step(const HimuonAdamwDesc* descs_dev, int n_descs,
                      int64_t n_chunks, int dtype, const double* beta1_by_group,
                      const double* beta2_by_group, const double* eps_by_group,
                      int n_groups, float* bias_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HIMUON_HIP_H */
