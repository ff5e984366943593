/*
 * enchip.h -- C ABI of libenchip.so, the MI355X (gfx950) W8A8 linear engine that
 * aikit's encoder reaches through a "hip" backend.
 *
 * The Go leaf `gpu/enchip` binds these symbols with purego (dlopen, no cgo) and
 * implements encoder.Backend / encoder.Q8Backend / W8A8Backend on top of them,
 * registering with encoder.RegisterBackend("hip", ...) from init(). Plain C types
 * only: no C++ or torch types cross this boundary.
 *
 * Conventions
 *   - Every entry point returns an int status: ENCHIP_OK (0) means handled; any
 *     other value means the call did nothing useful and the caller must fall back
 *     to its CPU path (the reference seam's "decline", encoder/backend_use.go:77-80).
 *     enchip_last_error() then describes the failure.
 *   - Matrices are row-major. a[M,K] f32 activations, wq[N,K] int8 weights in the
 *     PyTorch [out,in] layout, wscale[N], dst[M,N] f32, bias[N] (nullable).
 *   - Host pointers are borrowed for the duration of the call only.
 *   - A context owns all device memory it allocates; enchip_close frees it.
 *   - Every entry point takes a per-context mutex, so a context may be called from
 *     several threads at once (encoder.EncodeBatch's worker goroutines,
 *     encoder/model.go:214; enccuda serialises the same way,
 *     gpu/enccuda/backend.go:87,141-142). Host-pointer entry points are synchronous.
 *   - The context's device scratch (the quantized activations of the entry points
 *     that quantize themselves, the top-k candidates) is shared by all of them. Work
 *     that uses it on one stream waits, on the device, for its last use on another
 *     stream (an event the library records after each such use), so host calls and
 *     *_dev calls on different streams may be mixed. Under HIP graph capture the
 *     library records no such event and the caller orders the streams.
 *
 * Numerics (bit-exact against aikit's Go linalg path, default amd64 build):
 *   codes   = quantizeRowInt8Core (linalg/quant.go:43-71), activations' zero row -> scale 0
 *   acc     = exact int32 dot                      (linalg/quant.go:150-156)
 *   y       = float32(acc) * aScale[m] * wScale[n] (linalg/quant.go:295), +0 when aScale[m]==0
 *   y      += bias[n]                              (encoder/linalg.go:130-140)
 *   y       = GELUF32(y) when act == ENCHIP_ACT_GELU (linalg/exp.go:260-263)
 */
#ifndef ENCHIP_H
#define ENCHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ENCHIP_ABI_VERSION 3

typedef struct enchip_ctx enchip_ctx;
typedef uint64_t enchip_weight; /* opaque handle; 0 is never a valid handle */

enum enchip_status {
    ENCHIP_OK = 0,
    ENCHIP_ERR_NO_DEVICE = 1, /* no HIP device, or the device index is out of range */
    ENCHIP_ERR_ARG = 2,       /* invalid argument (null pointer, bad shape, K mismatch) */
    ENCHIP_ERR_HIP = 3,       /* a HIP runtime call failed */
    ENCHIP_ERR_OOM = 4,       /* device allocation failed */
    ENCHIP_ERR_HANDLE = 5     /* unknown or released weight handle */
};

enum enchip_act {
    ENCHIP_ACT_NONE = 0,
    ENCHIP_ACT_GELU = 1, /* exact-erf GELU, linalg.GELUF32 */
    ENCHIP_ACT_TANH = 2  /* linalg.TanhF32; enchip_bias_act_rows_dev only */
};

/* Layout of the b operand of enchip_matmul_bt_f32_dev. */
enum enchip_b_layout {
    ENCHIP_B_NK = 0, /* b[N, K] rows, pitch ldb: MatmulBT's own b (dst = a . b^T) */
    ENCHIP_B_KN = 1  /* b[K, N] rows, pitch ldb: dst = a . b, e.g. V for scores . V */
};

/* Returns ENCHIP_ABI_VERSION. Lets a binding check it loaded the library it was
 * written against before calling anything else. No reference counterpart. */
int enchip_abi_version(void);

/* Opens device `device` and creates a context with its own HIP stream.
 * Replaces enccuda.New -> gpu.CreateSystemDefaultDevice -> dev.NewViT
 * (gpu/enccuda/backend.go:97-101; gpu/cuda.go:87-100; gpu/cuda_vit.go:174-208):
 * device bring-up, kernel load and queue creation.
 * On failure *out is NULL and enchip_last_error(NULL) says why. */
int enchip_open(int device, enchip_ctx **out);

/* Frees every device buffer and weight the context owns. Idempotent on NULL.
 * Replaces Backend.Close (encoder/backend.go:26-27; gpu/enccuda/backend.go). */
int enchip_close(enchip_ctx *ctx);

/* The message of the calling thread's last failed call on ctx (the context's most
 * recent message when this thread has had none; for ctx == NULL, that of the last
 * failed enchip_open on this thread). Never NULL. The text is a copy owned by the
 * calling thread, valid until its next enchip_last_error call, so a failure on another
 * thread cannot replace or free it. A Go caller reads it on the OS thread that made the
 * failed call (runtime.LockOSThread around the pair). Diagnostics only. */
const char *enchip_last_error(const enchip_ctx *ctx);

/* Device facts used for roofline reporting: compute-unit count, peak engine clock
 * in kHz, and the gfx architecture name (e.g. "gfx950"). name_len includes the NUL.
 * Replaces the device queries behind gpu/roofline_test.go:57-140. */
int enchip_device_info(enchip_ctx *ctx, int *num_cus, int *clock_khz, char *name,
                       int name_len);

/* Per-row dynamic symmetric int8 quantization of a[M,K] into aq[M,K] and
 * ascale[M], on the device, host buffers in and out. Replaces
 * linalg.QuantizeActivationsInto (linalg/quant.go:206-213; all-zero row ->
 * scale 0) and the CUDA quant_rows kernel (gpu/vit.cu:49-83). */
int enchip_quant_rows(enchip_ctx *ctx, const float *a, int64_t M, int64_t K,
                      int8_t *aq, float *ascale);

/* Uploads an int8 weight matrix wq[N,K] with per-output-channel scales wscale[N]
 * once, pre-swizzled into the MFMA operand layout, and returns a handle. The
 * context keeps its own copy: the caller may free wq/wscale afterwards. Replaces
 * the (ptr,len)-keyed weight residency of gpu/enccuda/backend.go:204-244 for
 * linalg.WeightMat{w8a8: true} (linalg/weightmat.go:61-64,117-118). */
int enchip_weight_register(enchip_ctx *ctx, const int8_t *wq, const float *wscale,
                           int64_t N, int64_t K, enchip_weight *out);

/* Releases a registered weight's device memory. */
int enchip_weight_release(enchip_ctx *ctx, enchip_weight w);

/* Pre-swizzled weight images: the device's fragment-major layout of an N x K int8
 * weight, byte (n, k) at ((n/32)*(Kp/32) + k/32)*1024 + ((n%32) + 32*((k/16)%2))*16 + k%16
 * with Np = N rounded up to 256 and Kp = K rounded up to 64 (padding zero), so a model
 * converted once can be registered straight from a memory-mapped file without the
 * per-byte host swizzle: the device side of loading pre-quantized int8 weights from a
 * mapping (linalg.WrapInt8 / WeightMat.MappedSpan, linalg/weightmat.go:81-88,215-231;
 * embed.OpenSafetensorsMmap, embed/safetensors.go:290-305).
 *
 * enchip_weight_image_bytes: Np * Kp, or -1 for a shape enchip_weight_register refuses.
 * enchip_weight_export: copies weight w's image (image_bytes must be exactly its size)
 * and, when wscale is not NULL, its N scales back to the host.
 * enchip_weight_register_image: registers an image (and N scales) as
 * enchip_weight_register would have built it; refuses an image of the wrong size. */
int64_t enchip_weight_image_bytes(int64_t N, int64_t K);
int enchip_weight_export(enchip_ctx *ctx, enchip_weight w, int8_t *image, int64_t image_bytes,
                         float *wscale);
int enchip_weight_register_image(enchip_ctx *ctx, const int8_t *image, int64_t image_bytes,
                                 const float *wscale, int64_t N, int64_t K, enchip_weight *out);

/* Shape of a registered weight. */
int enchip_weight_shape(enchip_ctx *ctx, enchip_weight w, int64_t *N, int64_t *K);

/* One W8A8 linear on host buffers, synchronous:
 *   dst[M,N] = act(W8A8(a[M,K], w) + bias)
 * i.e. linalg.MatmulBTW8A8Into (linalg/quant.go:192-234) followed by addBias
 * (encoder/linalg.go:130-140) and, for ENCHIP_ACT_GELU, gelu
 * (encoder/bert.go:397-413). bias may be NULL. When acc_debug is non-NULL the
 * int32 accumulators [M,N] are also written to it (parity testing).
 * This is the body of the new opt-in W8A8Backend.MatmulBTW8A8 capability; the
 * weight-only Q8Backend.MatmulBTQ8 contract (encoder/backend_use.go:59-83) is NOT
 * served by it (enchip_matmul_bt_q8 serves that one). */
int enchip_w8a8_linear(enchip_ctx *ctx, enchip_weight w, const float *a, int64_t M,
                       const float *bias, int act, float *dst, int32_t *acc_debug);

/* The shared-activation batch: one quantization of a[M,K], then nops linears, each
 * with its own weight, bias, activation and dst[M, N_i]. Numerically identical to
 * calling enchip_w8a8_linear once per op. Replaces linalg.MatmulBTW8A8Batch /
 * W8A8Op (linalg/quant.go:303-370): BERT's Q,K,V projections share one quant. */
typedef struct enchip_op {
    enchip_weight w;
    const float *bias; /* nullable */
    int act;
    float *dst; /* [M, N of w] */
} enchip_op;
int enchip_w8a8_batch(enchip_ctx *ctx, const float *a, int64_t M, int64_t K,
                      const enchip_op *ops, int nops);

/* ---- device-resident entry points (pointers are device memory) ----------------
 * stream is a hipStream_t (NULL = the context's own stream). They enqueue work and
 * return without synchronising. No reference counterpart: the reference seam
 * passes host slices per call (encoder/backend.go:19-28); these are the resident
 * form the seam's planned residency widening needs (docs/task-native-gpu.md:418-427). */

/* Device form of enchip_quant_rows: d_a[M,K] row-major f32 in; codes out at row
 * pitch ldq >= K (columns [K,ldq) are written as zero), d_ascale[M].
 * linalg.QuantizeActivationsInto (linalg/quant.go:206-213). With ldq a multiple of
 * 64 the result feeds enchip_w8a8_pre_dev directly. */
int enchip_quant_rows_dev(enchip_ctx *ctx, const float *d_a, int64_t M, int64_t K,
                          int8_t *d_aq, int64_t ldq, float *d_ascale, void *stream);

/* GEMM + fused epilogue on ALREADY quantized activations: d_aq[M][ldq] int8 with
 * ldq a multiple of 64, ldq >= K and columns [K,ldq) zero (as enchip_quant_rows_dev
 * writes them), d_ascale[M]. d_dst[M,N] = act(W8A8 + bias).
 * linalg.MatmulBTW8A8Pre (linalg/quant.go:215-234): quantize once, reuse across
 * weights. Bit-identical to enchip_w8a8_linear_dev on the same activations. */
int enchip_w8a8_pre_dev(enchip_ctx *ctx, enchip_weight w, const int8_t *d_aq,
                        int64_t ldq, int64_t M, const float *d_ascale,
                        const float *d_bias, int act, float *d_dst, void *stream);

/* Device form of enchip_w8a8_linear. d_bias may be NULL. When
 * enchip_frag_route(ctx, w, M) is 1 it runs exactly the kernels of
 * enchip_quant_rows_frag_dev + enchip_w8a8_pre_frag_dev. */
int enchip_w8a8_linear_dev(enchip_ctx *ctx, enchip_weight w, const float *d_a,
                           int64_t M, const float *d_bias, int act, float *d_dst,
                           void *stream);

/* enchip_w8a8_linear_dev with no device allocation: the same kernels and bits, but the
 * quantized activations and their scales go to a fixed per-device scratch array of the
 * library (32 MiB of codes + 2^18 row scales, held by each device the library runs on
 * until the process ends) instead of the context's growable scratch, and the call makes
 * no hipMalloc / hipFree or other allocating call. No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). Declines with ENCHIP_ERR_ARG when M > 2^18 or the
 * codes (M rounded up to 128 rows when the persistent GEMM runs, else M, times K
 * rounded up to 64) exceed 32 MiB. Every call on a device shares that device's array
 * (across contexts and streams) and leaves its contents behind. Outside stream capture
 * the library orders the calls itself: each call's kernels wait on a per-device event
 * recorded after the previous call's (an event wait allocates nothing). Under capture
 * they do not (a graph cannot wait on an event recorded outside it), so captured calls
 * that overlap on one GPU race; the caller serialises them. */
int enchip_w8a8_linear_noalloc_dev(enchip_ctx *ctx, enchip_weight w, const float *d_a, int64_t M,
                                   const float *d_bias, int act, float *d_dst, void *stream);

/* Fragment-major twins of enchip_quant_rows_dev / enchip_w8a8_pre_dev (the same
 * reference interfaces, linalg/quant.go:206-234, with a device-native code layout).
 * The codes are laid out as the weights are: byte (r, k) of the M x ldq code matrix at
 *   ((r/32)*(ldq/32) + k/32)*1024 + ((r%32) + 32*((k/16)%2))*16 + k%16,
 * i.e. one 1 KiB block per 32 rows x 32 k in the operand order of
 * v_mfma_i32_32x32x32_i8, so the persistent GEMM loads 16 contiguous bytes per lane.
 * ldq must equal the weight's padded K (K rounded up to 64; enchip_frag_route checks
 * it is usable) and d_aq must hold roundup(M, 128) * ldq bytes: rows past M are read
 * by the GEMM but never stored, so their content is irrelevant. */
int enchip_quant_rows_frag_dev(enchip_ctx *ctx, const float *d_a, int64_t M, int64_t K,
                               int8_t *d_aq, int64_t ldq, float *d_ascale, void *stream);

/* enchip_quant_rows_frag_dev of GELU(d_a): the codes and scales it would write for the
 * rows d_a after linalg.GELUF32 (linalg/exp.go:260-263) on every element, computed from
 * the pre-activations d_a without writing the GELU outputs. Replaces the pair
 * "W8A8 linear with the GELU epilogue, then quantization of its output" in
 * encoder/bert.go:357-364 (intermediate = GELU(h Wi^T + bi); output = intermediate Wd^T
 * + bd): the first linear runs with act = ENCHIP_ACT_NONE and this call quantizes
 * GELU(its output) for the second, bit-identical to the pair. Requires K % 4 == 0,
 * ldq <= 4096 (else ENCHIP_ERR_ARG) and 16-byte aligned d_a and d_aq; otherwise the
 * layout and sizes of enchip_quant_rows_frag_dev. */
int enchip_quant_rows_frag_gelu_dev(enchip_ctx *ctx, const float *d_a, int64_t M, int64_t K,
                                    int8_t *d_aq, int64_t ldq, float *d_ascale, void *stream);

/* GEMM + fused epilogue on fragment-major codes from enchip_quant_rows_frag_dev.
 * Returns ENCHIP_ERR_ARG unless enchip_frag_route(ctx, w, M) is 1. Bit-identical to
 * enchip_w8a8_pre_dev / enchip_w8a8_linear_dev on the same activations. */
int enchip_w8a8_pre_frag_dev(enchip_ctx *ctx, enchip_weight w, const int8_t *d_aq,
                             int64_t ldq, int64_t M, const float *d_ascale,
                             const float *d_bias, int act, float *d_dst, void *stream);

/* 1 when a linear on weight w with M rows runs the persistent GEMM on fragment-major
 * codes (M above the small-M limit, N % 4 == 0, an even number of 64-deep K stages,
 * 32-bit offsets), else 0; the padded K (the ldq the frag entry points take) goes to
 * *ldq when ldq is not NULL. No reference counterpart: it exposes a dispatch choice. */
int enchip_frag_route(enchip_ctx *ctx, enchip_weight w, int64_t M, int64_t *ldq);

/* Name of the GEMM kernel instantiation a linear on weight w with M rows and
 * activation act launches (as it appears in rocprofv3 traces) when it quantizes its own
 * 16-byte aligned activations (enchip_w8a8_linear_dev; at small M that is the single
 * quantize + GEMV kernel), written to buf
 * (NUL-terminated, truncated to len). Diagnostics for attributing profiles to
 * calls; no reference counterpart. */
int enchip_gemm_kernel_name(enchip_ctx *ctx, enchip_weight w, int64_t M, int act,
                            char *buf, int len);

/* Measured device ceilings (best of 5): HBM streaming read (the best of 8 or 16 16-byte
 * loads in flight per lane and two grid sizes) and write over a 1 GiB buffer (past the
 * 256 MiB MALL); the dense int8 MFMA rate (v_mfma_i32_32x32x32_i8, 8 independent chains per
 * wave, 2 blocks per CU) twice: with constant operands, and with a different pair of
 * bell-shaped int8 operand fragments (standard deviation ~37, like quantized normal data)
 * in every instruction, each with the mean shader clock its blocks ran at (s_memtime over
 * s_memrealtime): the chip lowers its clock under the multipliers' power on real data;
 * and the f32 VALU rate in lane-operations per second for unfused, unpacked multiplies and
 * adds (8 independent chains per lane, 8 waves per SIMD): the roof of the bit-exact
 * epilogues, which are made of exactly those.
 * Replaces gpu/roofline.cu's stream_read / imad_peak / dp4a_peak probes and
 * TestDeviceCeilings (gpu/roofline_test.go:57-140). Allocates and frees 1 GiB. */
typedef struct enchip_ceilings {
    double hbm_read_gbps;
    double hbm_write_gbps;
    double mfma_i8_tops;      /* constant operands */
    double valu_f32_tops;     /* T lane-operations / s */
    double mfma_i8_mhz;       /* shader clock during the constant-operand MFMA probe */
    double mfma_i8_data_tops; /* bell-shaped random operands */
    double mfma_i8_data_mhz;  /* shader clock during that probe */
} enchip_ceilings;
int enchip_probe_ceilings(enchip_ctx *ctx, enchip_ceilings *out);

/* f32 dst[M,N] = a[M,K] . b[N,K]^T on host buffers, all row-major: the device side of
 * encoder.Backend.MatmulBT (encoder/backend.go:19-28; enccuda's MatmulBT,
 * gpu/enccuda/backend.go:136-172). Synchronous. a and b are uploaded on every call
 * (their contents are never cached: attention rewrites the same pooled buffers
 * between calls), dst is downloaded before returning. Products and sums are f32 on
 * the f32 MFMA in an order of its own; the contract is the reference's gate, worst
 * |dst - float64 dot| / max(|float64 dot|, 1) <= 2e-4 (gpu/enccuda/backend_test.go:
 * 47-86). K == 0 gives zeros. Which shapes are worth the round trip is the caller's
 * choice (enccuda's minGPUFlops, gpu/enccuda/backend.go:48-75): this entry point
 * always runs on the device. */
int enchip_matmul_bt_f32(enchip_ctx *ctx, const float *a, const float *b, float *dst,
                         int64_t M, int64_t K, int64_t N);

/* One level of batching for enchip_matmul_bt_f32_dev: `count` problems, the next one's
 * operands `stride_a` / `stride_b` / `stride_c` floats further on. */
typedef struct enchip_f32_batch {
    int64_t count;
    int64_t stride_a, stride_b, stride_c;
} enchip_f32_batch;

/* Device form of enchip_matmul_bt_f32, batched over two levels and strided, enqueued on
 * `stream` (NULL: the context stream). For problem (i, o), i < inner->count,
 * o < outer->count (a NULL level is one problem):
 *   C[m][n] = sum_k A[m][k] * B(n, k) with A = d_a + i*inner->stride_a + o*outer->stride_a
 *   (pitch lda), C likewise from d_c (pitch ldc), B likewise from d_b with element (n, k)
 *   at B[n*ldb + k] (ENCHIP_B_NK) or B[k*ldb + n] (ENCHIP_B_KN).
 * Pitches and strides are in floats. One call covers every (head, sequence) of an
 * attention layer with the heads read in place from the [tokens, 3D] QKV rows: QK^T is
 * A = Q head (lda = 3D, inner stride hd, outer stride L*3D), B = K head (ENCHIP_B_NK);
 * scores . V is A = scores, B = V head (ENCHIP_B_KN) -- the reference's qH / kH / vHT
 * extraction (encoder/attention.go:95-111) without the copies. Same arithmetic and
 * contract as enchip_matmul_bt_f32; M, N, K, counts <= 2^30 and M*N <= 2^36. */
int enchip_matmul_bt_f32_dev(enchip_ctx *ctx, const float *d_a, int64_t lda, const float *d_b,
                             int64_t ldb, int b_layout, float *d_c, int64_t ldc, int64_t M,
                             int64_t K, int64_t N, const enchip_f32_batch *inner,
                             const enchip_f32_batch *outer, void *stream);

/* Weight-only int8 product with f32 activations on host buffers:
 *   dst[m][n] = sum_k a[m][k] * (f32(wq[n][k]) * wscale[n]),
 * the device side of encoder.Q8Backend.MatmulBTQ8 (encoder/backend_use.go:59-83; enccuda's
 * MatmulBTQ8, gpu/enccuda/backend.go:246-287, and the CPU path it stands in for,
 * encoder/scratch.go:211-218 -> matmulBTQ8Into, encoder/linalg_q8.go:80-84). w is a weight
 * registered by enchip_weight_register (or _register_image): the same int8 codes and scales
 * the W8A8 entry points use, resident on the device in int8, never widened in memory.
 * a[M,K] and dst[M,N] are row-major host buffers; a is uploaded on every call, dst
 * downloaded before returning. The activations are NEVER quantized: each is split
 * exactly into three bf16 parts and every product with a weight code is exact on the bf16
 * MFMA, summed in f32 in an order of its own, and the sum is multiplied by wscale[n] once.
 * The contract is the reference's gate against a float64 dot product, worst
 * |dst - ref| / max(|ref|, 1) <= 2e-4 (gpu/enccuda/backend_test.go:234-289). K == 0 gives
 * zeros. A weight with an infinite scale is refused (ENCHIP_ERR_ARG): the CPU path
 * scales each code before the sum and gets NaN where a code is 0, which a scale applied
 * to the sum cannot reproduce. Which shapes are worth the round trip is the caller's
 * choice (enccuda's minGPUFlops): this entry point always runs on the device.
 * M <= 2^30, M*N <= 2^36. */
int enchip_matmul_bt_q8(enchip_ctx *ctx, enchip_weight w, const float *a, int64_t M,
                        float *dst);

/* Device form of enchip_matmul_bt_q8: d_a[M,K] with row pitch lda >= K and d_dst[M,N]
 * with row pitch ldd >= N, in floats, on device buffers, enqueued on `stream` (NULL: the
 * context stream). Same arithmetic and contract; allocates nothing. */
int enchip_matmul_bt_q8_dev(enchip_ctx *ctx, enchip_weight w, const float *d_a, int64_t lda,
                            int64_t M, float *d_dst, int64_t ldd, void *stream);

/* The f32 row operations between a BERT layer's linears, in place on device buffers,
 * enqueued on `stream` (NULL: the context stream). Each restates the reference operation
 * for operation; softmax and LayerNorm add their float64 partial sums as a tree across
 * a wavefront, so their float64 sums may differ from the reference's left-to-right
 * order in the last bits (an output, rarely, by one f32 ulp).
 *
 * Softmax of each of `rows` rows of `cols` floats (pitch ld), scaled first:
 * linalg.SoftmaxRowScaledInto (linalg/exp.go:174-182, exp_scalar.go:9-35,84-89) as
 * attention applies it to QK^T (encoder/attention.go:109). cols <= 4096. */
int enchip_softmax_rows_scaled_dev(enchip_ctx *ctx, float *d_x, int64_t ld, int64_t rows,
                                   int64_t cols, float scale, void *stream);

/* h = layerNorm(h + y) per row: the f32 residual add of encoder/attention.go:123-127 and
 * encoder/bert.go:363-365 (d_y may be NULL: no residual), then encoder/layernorm.go:18-38
 * (float64 mean and variance, divisor D, gain d_w[D], shift d_b[D]). D <= 4096. */
int enchip_residual_layer_norm_dev(enchip_ctx *ctx, float *d_h, int64_t ldh, const float *d_y,
                                   int64_t ldy, int64_t rows, int64_t D, const float *d_w,
                                   const float *d_b, double eps, void *stream);

/* enchip_residual_layer_norm_dev fused with the next linear's quantization: h = LN(h + y)
 * in place, exactly as enchip_residual_layer_norm_dev computes and stores it, and the
 * stored rows quantized per token into fragment-major codes + scales exactly as
 * enchip_quant_rows_frag_dev(d_h, rows, D, d_aq, ldq, d_ascale) would then produce them
 * (same layout and contract: ldq the weight's padded K, d_aq holding roundup(rows, 128)
 * * ldq bytes). The pair's output feeds enchip_w8a8_pre_frag_dev; the normalised rows are
 * not read back from device memory. No reference counterpart as one call: it is the
 * encoder/bert.go:352-353,363-367 residual + layerNorm followed by the quantization of
 * linalg.MatmulBTW8A8 (linalg/quant.go:43-71) for the next layer's linear. D a multiple
 * of 4, h, y, w, b, aq 16-byte aligned, D <= ldq <= 4096. */
int enchip_residual_layer_norm_quant_dev(enchip_ctx *ctx, float *d_h, int64_t ldh,
                                         const float *d_y, int64_t ldy, int64_t rows,
                                         int64_t D, const float *d_w, const float *d_b,
                                         double eps, int8_t *d_aq, int64_t ldq,
                                         float *d_ascale, void *stream);

/* BERT's embedding rows on the device (encoder/bert.go:299-322, before its LayerNorm):
 * for token i of each of nseq sequences of L tokens (d_ids[z*L + i]),
 *   h = word[clampTokenID(id)] + pos[i + pos_off]   then, when type_vocab > 0,
 *   h += type[seg], seg = d_segs[z*L + i] (0 when d_segs is NULL or seg is outside
 *   [0, type_vocab)),
 * f32 adds column by column in that order, so the rows are bit-identical to the
 * reference's. clampTokenID (encoder/forward.go:15-20): an id outside [0, vocab) reads
 * row 0. Tables are row-major [rows][D]; pos has npos rows and L + pos_off <= npos
 * (pos_off 0 for BERT, pad_token_id + 1 for RoBERTa / XLM-R). Row z*L + i goes to
 * d_h + (z*L + i)*ldh. The embedding LayerNorm is enchip_residual_layer_norm_dev with
 * d_y = NULL. */
int enchip_embed_rows_dev(enchip_ctx *ctx, const int32_t *d_ids, const int32_t *d_segs,
                          int64_t nseq, int64_t L, const float *d_word, int64_t vocab,
                          const float *d_pos, int64_t npos, int64_t pos_off,
                          const float *d_type, int64_t type_vocab, int64_t D, float *d_h,
                          int64_t ldh, void *stream);

/* x = act(x + bias) in place on rows x cols (pitch ld; d_bias[cols] may be NULL), act
 * ENCHIP_ACT_NONE or ENCHIP_ACT_TANH (linalg.TanhF32, linalg/exp.go:319-337, with
 * linalg.ExpF32's guards): the cross-encoder head's addBias + TanhInto after the pooler
 * and addBias after the classifier (encoder/crossencoder.go:229-236). Bit-identical to
 * the reference's f32 operations. */
int enchip_bias_act_rows_dev(enchip_ctx *ctx, float *d_x, int64_t ld, int64_t rows, int64_t cols,
                             const float *d_bias, int act, void *stream);

/* Mean pooling then L2 normalisation of nseq sequences of L rows each (rows
 * z*L .. z*L+L-1 of d_h, pitch ldh) into d_out[nseq][ldo]: encoder/pooling.go:84-105
 * poolOne(mean) and embed/pool.go:22-38 L2Normalize, in their summation order, so the
 * result is exact. L == 0 gives zero vectors, as the reference does. D <= 4096,
 * nseq <= 65535. */
int enchip_pool_mean_l2_dev(enchip_ctx *ctx, const float *d_h, int64_t ldh, int64_t nseq,
                            int64_t L, int64_t D, float *d_out, int64_t ldo, void *stream);

/* Scaled dot-product attention on device buffers, every head of nseq sequences of L
 * tokens in one call: encoder/attention.go:81-121 attentionCore (mOut = L) up to the
 * context, ctx = softmaxRowScaled(Q_h . K_h^T, scale) . V_h per head, written into
 * d_out's head columns. Row i of sequence z, head h of Q starts at
 * d_q + (z*L + i)*ld + h*head_dim (likewise K, V; all three share the pitch, as in the
 * fused [tokens, 3D] QKV rows) and the context at d_out + (z*L + i)*ldo + h*head_dim.
 * The score tile of 32 queries stays in on-chip memory (never written to device
 * memory); its softmax and products run as set by enchip_set_attention_products, and the
 * result agrees with enchip_matmul_bt_f32_dev + softmax + matmul within the f32 MatmulBT
 * gate (gpu/enccuda/backend_test.go:71-81: <= 2e-4 of max(|ref|, 1); summation order
 * differs). head_dim 32 or 64; L <= 512 in the two-pass modes, any L in the default mode;
 * ld a multiple of 4; q, k, v 16-byte aligned. */
int enchip_attention_f32_dev(enchip_ctx *ctx, const float *d_q, const float *d_k,
                             const float *d_v, int64_t ld, float *d_out, int64_t ldo,
                             int64_t nseq, int64_t L, int64_t heads, int64_t head_dim,
                             float scale, void *stream);

/* How enchip_attention_f32_dev computes the attention (no reference counterpart: a
 * device tuning choice, like enchip_set_small_m):
 *   ENCHIP_ATT_FLASH_F16  (the default) one pass over the keys with an online softmax
 *                         (running maximum, 2^x on the hardware, the context rescaled as
 *                         the maximum grows, divided by the sum at the end), both products
 *                         on the f16 MFMA over operands split into two IEEE half parts
 *                         (x.y ~ hi.hi' + hi.lo' + lo.hi', each product within ~3 * 2^-22
 *                         of exact, summed in f32), K and V staged through on-chip memory
 *                         once per 256 queries. Any L. Within the f32 MatmulBT gate on
 *                         inputs of standard deviation up to 4 (tested). Operands must be
 *                         below 65520 in magnitude: larger ones give NaN.
 *   ENCHIP_ATT_FLASH_BF16 the same kernel with the operands split into bfloat16 parts
 *                         (each product within 3 * 2^-18): any finite operand, but 2^6
 *                         times the product error (above the gate at standard deviation 2).
 *   ENCHIP_ATT_SPLIT_BF16 the reference's two-pass softmax (enchip_softmax_rows_scaled_dev's
 *                         steps) on a 32-query score tile held on chip, bfloat16 split
 *                         products. L <= 512.
 *   ENCHIP_ATT_F32        the same two-pass kernel with f32 MFMA products
 *                         (v_mfma_f32_32x32x2_f32). L <= 512.
 * Non-finite operands give NaN in the split modes. Applies to later calls on this context. */
enum enchip_att_products {
    ENCHIP_ATT_F32 = 0,
    ENCHIP_ATT_SPLIT_BF16 = 1,
    ENCHIP_ATT_FLASH_BF16 = 2,
    ENCHIP_ATT_FLASH_F16 = 3
};
int enchip_set_attention_products(enchip_ctx *ctx, int mode);

/* The k best of each of `rows` rows of n scores (pitch ld), on the device:
 * ann.I8TopKIndex's selection (ann/backend.go:46-55), identical to FlatI8.topHits
 * (ann/flat_i8.go:208-242) on the same scores: score descending, equal scores by
 * ascending index (topk.Cmp, topk/cmp.go:15-27), NaN never retained
 * (topk/topk.go:93-100). Row r's i-th best goes to d_index[r*ldi + i] (its column in
 * [0, n)) and d_score[r*lds + i]; a row with fewer than k non-NaN scores pads with index
 * -1 and a NaN score (the reference returns the shorter list). The score matrix is read
 * once; candidates use the context's scratch. k <= 1024, n < 2^31. */
int enchip_topk_rows_dev(enchip_ctx *ctx, const float *d_scores, int64_t ld, int64_t rows,
                         int64_t n, int64_t k, int32_t *d_index, int64_t ldi, float *d_score,
                         int64_t lds, void *stream);

/* ann.I8TopKIndex.TopKBatch (ann/backend.go:46-55) on an index registered as a weight
 * (codes [n, dim], per-row scales): queries[M, dim] f32 on the host are quantized per
 * row, scored against every index row with the bias-free W8A8 linear
 * ("(float)acc*qscale*scale", ann/backend.go:25-29), and each query's k best hits come
 * back in hit_index[M, k] / hit_score[M, k] (as enchip_topk_rows_dev orders and pads
 * them). Only the M x k hits cross back to the host, not the M x n scores.
 * Synchronous. k <= 1024. */
int enchip_ann_topk(enchip_ctx *ctx, enchip_weight index, const float *queries, int64_t M,
                    int64_t k, int32_t *hit_index, float *hit_score);

/* How enchip_ann_topk has run on this context: *fused = calls that took the fused route
 * (M >= 8, k <= 64, an index of at least 131072 rows whose dimension
 * padded to 64 is an even multiple of 64, as the tiled GEMM takes it: each query's
 * bound from the k-th best score of the index's first 32768 rows, then one scoring pass
 * that keeps only the scores at or above it, so the M x n scores are never written);
 * *fallbacks = those of them that then ran the two-pass route because some query kept
 * more than 4096 scores, or 8192 for k > 32 (an index ordered so that later rows keep
 * scoring higher). Both routes give identical results. No reference counterpart: a
 * diagnostic. */
int enchip_ann_topk_stats(enchip_ctx *ctx, int64_t *fused, int64_t *fallbacks);

/* Caps each growable device scratch buffer of the context at `bytes` (0, the default:
 * no cap). A call that would grow scratch past the cap declines with ENCHIP_ERR_OOM
 * before doing any work, exactly as a failed device allocation does, so a deployment
 * can bound the memory a context takes beyond its weights, and a test can force the
 * out-of-memory decline of enccuda's gpuMatmul (gpu/enccuda/backend.go:148-153: a
 * device allocation failure falls back to the CPU path). Weights are not scratch.
 * No reference counterpart. */
int enchip_set_scratch_limit(enchip_ctx *ctx, int64_t bytes);

/* Rows at or below which the small-M (HBM-bound, split-K) kernel runs instead of
 * the tiled MFMA GEMM. Both produce identical bits; this only selects the kernel.
 * Mirrors the reference's dispatch knobs (linalg.SetParallelThreshold,
 * linalg/linalg.go:58-74). Default 32. */
int enchip_set_small_m(enchip_ctx *ctx, int64_t max_m);

#ifdef __cplusplus
}
#endif
#endif /* ENCHIP_H */
