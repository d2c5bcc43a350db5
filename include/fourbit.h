/*
 * fourbit.h -- C ABI of libfourbit.so, the MI355X (gfx950) fused 4-bit dequant-GEMV.
 *
 * The reference (jvap2/If_I_could_turn_back_time) has no packed 4-bit path; its
 * quantized linear layer dequantizes to fp32 and calls F.linear
 * (Python_Jenks_Test/Jenks_Tests/Quantization_Experiments/layers.py:33-38), and its
 * only native FFI is torch::Tensor-typed inline CUDA loaded with load_inline
 * (Python_Jenks_Test/Jenks_Tests/cuda_helpers.py:42-62, 187-211, 293-299).  Each entry
 * point below names the reference interface it replaces.
 *
 * Conventions
 *  - Plain pointers and sizes only; no torch types.  The caller allocates every
 *    buffer; the library never allocates device memory.
 *  - Every function returns 0 (FB_OK) or a negative fb_status; fb_strerror() maps it
 *    to text.  Argument validation runs on the host and needs no GPU.
 *  - GPU entry points launch asynchronously on the given hipStream_t (passed as void*)
 *    and never synchronise the device.
 *  - Re-entrant: the only global state is a once-initialised device-property cache.
 */
#ifndef FOURBIT_H
#define FOURBIT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FB_ABI_VERSION 1

typedef enum {
  FB_OK = 0,
  FB_ERR_NULL = -1,          /* a required pointer is NULL                         */
  FB_ERR_SHAPE = -2,         /* N, K or B out of range                             */
  FB_ERR_GROUP = -3,         /* group size not supported for the format / K % group */
  FB_ERR_FORMAT = -4,        /* unknown fmt                                        */
  FB_ERR_DTYPE = -5,         /* unsupported x / y dtype for the format             */
  FB_ERR_FWHT = -6,          /* fwht_block not a power of two in [2,4096] | K      */
  FB_ERR_ALIGN = -7,         /* pointer not 16-byte aligned                        */
  FB_ERR_WORKSPACE = -8,     /* workspace too small                                */
  FB_ERR_BATCH = -9,         /* batch size not supported by this entry point       */
  FB_ERR_VALUE = -10,        /* non-finite / non-integer / out-of-range packer input */
  FB_ERR_HIP = -11,          /* a HIP runtime call failed                          */
  FB_ERR_THREADS = -12,      /* nthreads < 1                                       */
  FB_ERR_LDS = -13,          /* activation does not fit the kernel's LDS budget    */
  FB_ERR_LEVELS = -14,       /* integer levels of one 128-group span > 16 values    */
  FB_ERR_SCRATCH = -15       /* shape needs more than fb_gemv_noalloc's fixed scratch */
} fb_status;

typedef enum { FB_FMT_GF4 = 0, FB_FMT_E2M1 = 1 } fb_fmt;
/* FB_DT_F64 is taken by the per-split SSD entry points (fb_jenks2_ssd_*) only. */
typedef enum { FB_DT_F16 = 0, FB_DT_BF16 = 1, FB_DT_F32 = 2, FB_DT_F64 = 3 } fb_dtype;

/* One quantized linear layer: y[B,N] = x[B,K] . W[N,K]^T. */
typedef struct {
  int32_t N;           /* out-features (rows of W)                                   */
  int32_t K;           /* in-features (reduction dim); multiple of 128               */
  int32_t B;           /* batch rows of x / y                                        */
  int32_t group;       /* 128 for GF4, 32 for E2M1                                   */
  int32_t fmt;         /* fb_fmt                                                     */
  int32_t fwht_block;  /* 0 = no rotation, else power of two in [2, 4096] dividing K
                          (x' = H x/sqrt(b)) */
  int32_t x_dtype;     /* fb_dtype of x: GF4 needs F16; E2M1 takes F16 or BF16       */
  int32_t y_dtype;     /* fb_dtype of y: F16, BF16 or F32                            */
} fb_shape_t;

int fb_abi_version(void);
const char* fb_strerror(int code);

/* Host-side checks of a shape (no GPU needed). */
int fb_validate(const fb_shape_t* s);

/* Bytes of the device weight stream (nibbles + codebooks/scales; rows padded to a
 * multiple of 16 and K to a multiple of 512 with zero bytes) for fb_to_device /
 * fb_gemv. */
size_t fb_device_bytes(const fb_shape_t* s);

/* Workspace bytes fb_gemv can use for this shape on the current device (0 for invalid
 * shapes):
 *  - B*K*2 (rounded up to 256) for rotated shapes with B*K >= 16384, where x is rotated
 *    once into the workspace by its own small kernel before the GEMV;
 *  - plus P*B*N*4 (rounded up to 256) where the GEMV runs its K-parts side by side (batch
 *    >= 2 over a long K whose staged x would need 3 or more K-slices on few row tiles, e.g.
 *    11008 -> 4096 at batch 16, P = 4; not where each wave staging the x of its own spans
 *    is faster, 4 or more spans per wave on at least as many row tiles as CUs): each
 *    part's fp32 sums, added by one more small kernel in part order.
 * The contents need no initialisation and are not kept between calls. */
size_t fb_workspace_bytes(const fb_shape_t* s);

/* ---------------------------------------------------------------------------------
 * Host packers.  They replace the reference's per-row fp32 quantizer state
 * (layers.py:23-31, s/Q/Theta/mask as dense fp32 tensors) and its Jenks break search
 * (cuda_helpers.py:151-211 + :378-395, k = 2, O(n^2) per array) with deterministic
 * multithreaded packers.  Outputs are the canonical formats:
 *   codes    uint8  [N, K/2]  element 2j in bits 3:0, element 2j+1 in bits 7:4
 *   codebook uint16 [N, K/128, 16] fp16 bit patterns, non-decreasing   (GF4)
 *   scales   uint8  [N, K/32]  E8M0, value 2^(s-127)                      (E2M1)
 * ------------------------------------------------------------------------------- */

/* GF4: per (row, 128-group) optimal 16-class 1-D partition (Fisher/Jenks DP over the
 * stable-sorted group, fp64 prefix sums, ties to the smallest break), centroid =
 * class mean rounded fp64->fp32->fp16.  Generalises Jenks_Optimization
 * (cuda_helpers.py:151-184) from 2 to 16 classes. */
int fb_quantize_gf4(const float* w, int32_t N, int32_t K, uint8_t* codes, uint16_t* codebook,
                    int32_t nthreads);

/* GF4 with a keep mask (uint8 [N,K], 0 = masked, NULL = none, i.e. fb_quantize_gf4).
 * Masked weights decode to exactly 0, as the reference's mask * s * (...) does
 * (layers.py:37, :43): in every group that has a masked entry, the kept values get
 * min(15, kept) Jenks classes and the codebook gains an exact-zero entry, placed after
 * the strictly negative centroids; entries past the last used one repeat it.  Masked
 * values are never read (they may be non-finite). */
int fb_quantize_gf4_masked(const float* w, const uint8_t* keep, int32_t N, int32_t K,
                           uint8_t* codes, uint16_t* codebook, int32_t nthreads);

/* Integer-level weights (levels fp32 [N,K], integer-valued; scale fp32 [N], > 0) as
 * GF4: per 128-group, lo = min level, code = level - lo, codebook[j] =
 * fp16_rne(fp32(scale[n] * (lo + min(j, hi - lo)))).  Exact up to the fp16 rounding
 * of scale * level.  This is the reference's own 4-bit weight: QuantLinear.commit
 * stores mask * s * round(Q + Theta) (layers.py:39-45, level = mask * round(...)) and
 * brecq's AdaRound quantizer returns clamp(mask * (W_floor + h), qmin, qmax) * delta
 * (brecq.py:81-92).  FB_ERR_LEVELS when a group spans more than 16 levels (the
 * reference's [-8, 8] can, rarely, in one group). */
int fb_pack_levels_gf4(const float* levels, const float* scale, int32_t N, int32_t K,
                       uint8_t* codes, uint16_t* codebook, int32_t nthreads);

/* E2M1 + E8M0 per 32-group (OCP MX v1.0): e = floor(log2 amax) - 2, codes by RNE with
 * saturation at +-6, amax = 0 -> scale byte 127.  Replaces the uniform grids of
 * brecq.py:13-56 / utils.py:313-339 for this format. */
int fb_quantize_e2m1(const float* w, int32_t N, int32_t K, uint8_t* codes, uint8_t* scales,
                     int32_t nthreads);

/* Offline weight rotation, in place: each K-block of each row becomes
 * w H_b / sqrt(b) (fp64 butterflies, one rounding to fp32).  No reference counterpart. */
int fb_fwht_rows_f32(float* w, int32_t N, int32_t K, int32_t block, int32_t nthreads);

/* Canonical (codes + codebook|scales) -> device weight stream of fb_device_bytes(s)
 * bytes (pure permutation / table transform, host memory), and its inverse. */
int fb_to_device(const uint8_t* codes, const void* meta, void* wdev, const fb_shape_t* s);
int fb_from_device(const void* wdev, uint8_t* codes, void* meta, const fb_shape_t* s);

/* Host decode of canonical codes + codebook|scales to fp32 [N,K] (exact).  Produces
 * the committed weight of QuantLinear.commit() (layers.py:39-45), which the reference
 * stores as mask*s*round(Q+Theta) in fp32. */
int fb_dequant_host(const uint8_t* codes, const void* meta, float* w_out, const fb_shape_t* s);

/* ---------------------------------------------------------------------------------
 * GPU entry points (hipStream_t passed as void*).  They launch on the calling thread's
 * current HIP device; the stream and every device pointer must belong to it.
 * ------------------------------------------------------------------------------- */

/* Fused dequant-GEMV, batch 1..16: y = x' . W^T with x' = FWHT_b(x) when fwht_block.
 * Replaces QuantLinear.forward's dequantize + F.linear pair (layers.py:33-38;
 * brecq.py:323-329 new_forward) and the reference's native linear_kernel_batch
 * (CUDA_C_Code/include/layers.h:9828-9839).  wdev is the fb_to_device stream in
 * device memory; x is [B,K] of x_dtype, y is [B,N] of y_dtype.
 * ws: device workspace (256-byte aligned) of fb_workspace_bytes(s) bytes, or NULL.  With it,
 * a rotated call of B*K >= 16384 values rotates x once into ws (one extra small kernel)
 * and runs the unrotated GEMV on it, and a split-K shape runs its K-parts side by side with
 * their sums in ws; without it (NULL, too small or misaligned) every workgroup rotates x in
 * its prologue and the K-parts run within one launch (K-slices in turn, or each wave
 * staging the x of its own spans), which gives the same results within the tolerance (each
 * plan is deterministic) and is slower for such shapes.  Calls that share a
 * workspace must not overlap.
 * A batch whose staged activations do not fit LDS at once (a 4096-wide rotation done in
 * the prologue keeps an fp32 copy of every batch row) runs as several launches over row
 * chunks, each streaming the weights; FB_ERR_LDS only when a single row does not fit. */
int fb_gemv(const void* wdev, const void* x, void* y, const fb_shape_t* s, void* ws,
            size_t ws_bytes, void* stream);

/* fb_gemv that allocates nothing and takes no workspace.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory around a call (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The once-per-call
 * rotation's scratch is a file-scope device array of 1 MiB per GPU (its address is looked
 * up once per device on the first call there, and the array lives until the process
 * ends): rotated calls of B*K > 524288 values return FB_ERR_SCRATCH.  No hipMalloc, hipFree
 * or allocating library call is made.  Every call on a GPU shares that GPU's array, so
 * calls that overlap on one GPU (several streams or host threads) race; serialise them.
 * Split-K shapes keep their parts' sums in the array after the rotated x where they fit.
 * Results equal fb_gemv's with a workspace bit for bit, except for split-K shapes whose sums
 * do not fit: those run their K-parts within one launch, as fb_gemv does without a
 * workspace, within the tolerance of fb_gemv's result. */
int fb_gemv_noalloc(const void* wdev, const void* x, void* y, const fb_shape_t* s,
                    void* stream);

/* The E2M1 GEMV on the matrix cores' native FP4 path, an opt-in alternative to fb_gemv for
 * unrotated E2M1 weights with BF16 x, batch 1..16 (others: FB_ERR_FORMAT / FB_ERR_DTYPE /
 * FB_ERR_FWHT / FB_ERR_BATCH).  Same operands and result layout as fb_gemv and the same
 * reference interface (QuantLinear.forward's dequantize + F.linear, layers.py:33-38, and
 * linear_kernel_batch, layers.h:9828-9839); the reference has no FP4 mode of its own.
 * x is split once per call (one small kernel, into ws) into two MX-E4M3 terms, each E4M3
 * values times a power of two per 32-value block; v_mfma_scale_f32_16x16x128_f8f6f4 then
 * multiplies the stored E2M1 codes and E8M0 scales by both terms, with no decode.  The two
 * terms hold a bf16 value exactly unless its 32-value block spans more than E4M3's exponent
 * range (values 2^14 or more below the block's largest lose low bits), so y differs from
 * fb_gemv's by the accumulation order, plus that loss where it occurs.  E8M0 byte 0 is
 * 2^-127 here (fb_dequant_host's value; fb_gemv decodes it to 0).
 * ws: device workspace, 256-byte aligned, of at least fb_mx_workspace_bytes(s) bytes
 * (required: FB_ERR_NULL / FB_ERR_ALIGN / FB_ERR_WORKSPACE otherwise): the split, then the
 * split-K parts' sums where the plan runs them side by side.  Calls that share a workspace
 * must not overlap. */
int fb_gemv_mx(const void* wdev, const void* x, void* y, const fb_shape_t* s, void* ws,
               size_t ws_bytes, void* stream);

/* Workspace bytes of fb_gemv_mx for this shape on the current device (0 for shapes it
 * does not take). */
size_t fb_mx_workspace_bytes(const fb_shape_t* s);

/* The split fb_gemv_mx makes of x (BF16 [B,K] on the device), into out (device, 256-byte
 * aligned, fb_mx_split_bytes(s) bytes), asynchronous on the stream.  Layout: for batch row
 * b and 128-value group g, 256 bytes at (b*K/128 + g)*256 -- the 128 E4M3 codes (OCP
 * e4m3fn) of term 0, then the 128 of term 1, in K order; from byte offset B*K*2 rounded up
 * to 256, 8 bytes per (b, g) -- the E8M0 scales of the group's four 32-value blocks for
 * term 0, then for term 1.  Term t rounds (nearest, ties to even) what the earlier terms
 * left of x, in units of its block's scale 2^e, e the smallest with the block's largest
 * magnitude <= 448 * 2^e (clamped to [-127, 127]; 0 for a block of zeros).  For callers
 * that reuse one split across layers that share their input (fb_gemv_mx_presplit). */
int fb_mx_split(const void* x, void* out, const fb_shape_t* s, void* stream);

/* Bytes of fb_mx_split's output (0 for shapes fb_gemv_mx does not take). */
size_t fb_mx_split_bytes(const fb_shape_t* s);

/* fb_gemv_mx on a split made by fb_mx_split (xs: device, 256-byte aligned), for layers that
 * share their input (q/k/v or gate/up projections): one split, then one of these per layer.
 * Same results as fb_gemv_mx on the same x when given a workspace of
 * fb_mx_presplit_workspace_bytes(s) bytes (the split-K parts' sums; 256-byte aligned); with
 * NULL such shapes run their K-slices in turn, within the tolerance of that result.  Calls
 * that share a workspace must not overlap.  The reference interface replaced is fb_gemv_mx's. */
int fb_gemv_mx_presplit(const void* wdev, const void* xs, void* y, const fb_shape_t* s,
                        void* ws, size_t ws_bytes, void* stream);

/* Workspace bytes of fb_gemv_mx_presplit (0: none used, or a shape it does not take). */
size_t fb_mx_presplit_workspace_bytes(const fb_shape_t* s);

/* GF4 packer on the GPU: the same arithmetic as fb_quantize_gf4 (keep == NULL) and
 * fb_quantize_gf4_masked, one wavefront per (row, 128-group), fp64; the outputs are
 * bit-identical to the host packers.  w fp32 [N,K], keep uint8 [N,K] or NULL, codes uint8
 * [N,K/2] and codebook uint16 [N,K/128,16] are device pointers (canonical layout; convert
 * with fb_to_device).  Asynchronous on the stream.  Non-finite kept weights are not
 * detected here (the host packers reject them): their group's output is unspecified, so
 * callers check first.  Replaces the reference's GPU Jenks search
 * (cuda_helpers.py:151-211, one thread per split of a 2-class problem) with the 16-class
 * DP. */
int fb_quantize_gf4_gpu(const float* w, const uint8_t* keep, int32_t N, int32_t K,
                        uint8_t* codes, uint16_t* codebook, void* stream);

/* E2M1 packer on the GPU: the same rule and bytes as fb_quantize_e2m1, 32 lanes per
 * 32-group.  w fp32 [N,K], codes uint8 [N,K/2] and scales uint8 [N,K/32] are device
 * pointers; asynchronous on the stream; non-finite weights are not detected here. */
int fb_quantize_e2m1_gpu(const float* w, int32_t N, int32_t K, uint8_t* codes, uint8_t* scales,
                         void* stream);

/* Device decode of the whole weight: w_out [N,K] of out_dtype (F32 always exact; F16
 * exact for GF4; BF16 exact for E2M1 within the bf16 normal range).  The same decode
 * code as fb_gemv; used for bit-exact parity.  Replaces the dequantizer expression
 * mask*s*(Q+Theta) (layers.py:36-37) / AdaRoundQuantizer.forward (brecq.py:81-92). */
int fb_dequant(const void* wdev, void* w_out, int32_t out_dtype, const fb_shape_t* s,
               void* stream);

/* ---------------------------------------------------------------------------------
 * Two-class natural breaks over a whole array (k = 2 Jenks): the reference's weight and
 * bias pruning masks, Linear_Mask / Bias_Mask (cuda_helpers.py:378-411), which call
 * jenks_optimization_cuda / jenks_optimization_biases_cuda (cuda_helpers.py:151-211,
 * :85-140; also CUDA_C_Code/include/layers.h:2424-2560).  The reference computes, for every
 * split index idx of the ascending-sorted values, the SSD of [0, idx) about its mean plus the
 * SSD of [idx, n) about its own (idx = 0: one class, "no split"), one O(n) thread per split,
 * then takes the first argmin and keeps the values at sorted positions >= idx.  Here the
 * class sums come from fp64 prefix sums: O(n) after the sort.
 *   w      fp32 [n] (any shape, flattened), finite
 *   keep   uint8 [n]: 1 where w[i] sits at a sorted position >= split (the reference's
 *          `arr[indices[var_min:]] = 1`), else 0
 *   split  int64: the first argmin over idx in [0, n)
 *   gvf    double: (ssd(0) - ssd(split)) / (ssd(0) + 1e-8), the reference's GVF
 * Arithmetic (fixed so host and GPU agree bit for bit): stable ascending sort (-0.0 ==
 * +0.0), c = sorted[n/2], d = sorted - c and d*d in fp64, prefix sums sequential within
 * blocks of 256, block totals sequential within superblocks of 256 blocks, superblock totals
 * sequential, ssd(i) = [i ? Q(i) - P(i)^2/i : 0] + [(Qt - Q(i)) - (Pt - P(i))^2/(n - i)].
 * The reference's own fp32 serial sums round differently: splits whose SSDs differ by less
 * than that rounding may be chosen differently.  1 <= n <= 2^31 - 1.
 * ------------------------------------------------------------------------------- */
int fb_jenks2_host(const float* w, int64_t n, uint8_t* keep, int64_t* split, double* gvf);

/* Device workspace bytes fb_jenks2_gpu needs for n values.  Queries the radix sort of the
 * current HIP device, so it needs a GPU (FB_ERR_HIP without one). */
int fb_jenks2_workspace(int64_t n, size_t* bytes);

/* GPU version of fb_jenks2_host, bit-identical outputs.  w, keep, split, gvf and ws are
 * device pointers (ws 256-byte aligned, at least fb_jenks2_workspace(n) bytes); asynchronous
 * on the stream.  Non-finite values are not detected here (fb_jenks2_host rejects them with
 * FB_ERR_VALUE), so callers check first. */
int fb_jenks2_gpu(const float* w, int64_t n, uint8_t* keep, int64_t* split, double* gvf,
                  void* ws, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * The same two-class split on every filter of a convolution weight on its own.  Replaces
 * the reference's Conv_Mask (Python_Jenks_Test/Jenks_Tests/cuda_helpers.py:333-376) over its
 * per-filter kernel jenks_optimization_cuda_conv (:219-289: one thread per (out, in) filter
 * pair trying every split of the kh*kw values serially, O(n^2) per filter).
 *   w      fp32 [nf, n]: filter f is w[f*n .. f*n + n), the (out, in) slices of an
 *          [out, in, kh, kw] weight (nf = out*in, n = kh*kw), finite
 *   keep   uint8 [nf, n]: fb_jenks2_host's mask of each filter
 *   split  int32 [nf]: each filter's first argmin over idx in [0, n)
 *   gvf    double [nf]: each filter's GVF
 * Each filter's split, GVF and mask are bit for bit what fb_jenks2_host gives on that
 * filter alone.  1 <= n <= FB_JENKS2_FILTER_MAX (a 32x32 kernel), 1 <= nf < 2^31.
 * ------------------------------------------------------------------------------- */
#define FB_JENKS2_FILTER_MAX 1024
int fb_jenks2_filters_host(const float* w, int64_t nf, int32_t n, uint8_t* keep, int32_t* split,
                           double* gvf, int32_t nthreads);

/* GPU version, bit-identical to fb_jenks2_filters_host: stable ranks by counting and the
 * fp64 sums in the host's order, one filter per lane for 1024 or more filters of at most 25
 * values, else one filter per one-wave workgroup; no workspace.  w, keep, split and gvf are
 * device pointers; asynchronous on the stream.  Non-finite values are not detected (the
 * host version rejects them with FB_ERR_VALUE). */
int fb_jenks2_filters_gpu(const float* w, int64_t nf, int32_t n, uint8_t* keep, int32_t* split,
                          double* gvf, void* stream);

/* ---------------------------------------------------------------------------------
 * The per-split SSD of arrays that arrive sorted, the interface the reference's optimizers
 * bind directly: var = module_weights.jenks_optimization_cuda(sorted) and
 * module_bias.jenks_optimization_biases_cuda(sorted), then var.argmin()
 * (Python_Jenks_Test/Jenks_Tests/custom_optimizer.py:135-136, :164-165 and 20 more sites),
 * over the kernels at cuda_helpers.py:151-211 and :85-146 (one thread per split, each
 * summing both classes serially: O(n^2)).  Here the prefix-sum rule of fb_jenks2_host, in
 * O(n), without its sort (the values are taken in the order given, as the reference's
 * kernels take them):
 *   sorted  fp32 or fp64 [n] (dtype FB_DT_F32 / FB_DT_F64), ascending as the caller sorted it
 *   ssd     [n] of the same dtype: ssd[i] = the within-class SSD of [0, i) plus that of
 *           [i, n) (i = 0: one class), fp64 sums in fb_jenks2_host's order, rounded to dtype
 * The reference's own serial fp32 (or fp64) two-pass sums round differently: values agree
 * to within that rounding (about 1e-5 of ssd[0] in fp32), and argmin agrees wherever the
 * minimum is not a near-tie.  Non-finite values give non-finite SSDs, as the reference's
 * do.  1 <= n <= 2^31 - 1.
 * ------------------------------------------------------------------------------- */
int fb_jenks2_ssd_host(const void* sorted, int64_t n, int32_t dtype, void* ssd);

/* Device workspace bytes fb_jenks2_ssd_gpu needs for n values (host-side arithmetic). */
int fb_jenks2_ssd_workspace(int64_t n, size_t* bytes);

/* GPU version of fb_jenks2_ssd_host, bit-identical.  sorted, ssd (16-byte aligned) and ws
 * (256-byte aligned, at least fb_jenks2_ssd_workspace(n) bytes) are device pointers;
 * asynchronous on the stream (the reference synchronises the device after its launch). */
int fb_jenks2_ssd_gpu(const void* sorted, int64_t n, int32_t dtype, void* ssd, void* ws,
                      size_t ws_bytes, void* stream);

/* The same per filter: module_conv.jenks_optimization_cuda_conv(sorted) (cuda_helpers.py:
 * 258-289 over the kernel at :219-255, called from Conv_Mask :356), whose input is an
 * [C0, C1, kh, kw] weight with each (c0, c1) filter's kh*kw values sorted, and whose output
 * is the SSD of every split of every filter, flat [C0*C1*kh*kw] in the same order.
 *   sorted  [nf, n] (nf = C0*C1 filters of n = kh*kw values), ssd [nf, n], same dtype;
 *   each filter's row is bit for bit fb_jenks2_ssd_host of that filter alone.
 * 1 <= n <= FB_JENKS2_FILTER_MAX, 1 <= nf < 2^31. */
int fb_jenks2_ssd_filters_host(const void* sorted, int64_t nf, int32_t n, int32_t dtype,
                               void* ssd, int32_t nthreads);

/* GPU version, bit-identical to fb_jenks2_ssd_filters_host: one thread per filter, no
 * workspace.  Device pointers aligned to the dtype's size; asynchronous on the stream. */
int fb_jenks2_ssd_filters_gpu(const void* sorted, int64_t nf, int32_t n, int32_t dtype,
                              void* ssd, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* FOURBIT_H */
