// enchip.hip -- libenchip.so: the C ABI declared in include/enchip.h.
//
// Context = one device + one HIP stream + registered weights + growable device
// scratch. Host-pointer entry points are synchronous and serialised by the
// context mutex; *_dev entry points only enqueue.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "enchip.h"
#include "attention_f32.h"
#include "attention_flash.h"
#include "encoder_ops.h"
#include "gemm_f32.h"
#include "gemm_persistent.h"
#include "gemm_q8w.h"
#include "gemm_skinny.h"
#include "topk.h"
#include "kernels.h"
#include "probes.h"

namespace {

constexpr int64_t kMaxK = 131072;  // K*127*127 stays below 2^31: the int32 dot cannot wrap
constexpr int64_t kRowPad = 256;   // quantized-activation scratch rows are padded to this
constexpr int64_t kColPad = 256;   // weight output channels are padded to this

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

struct Weight {
    int8_t *d_w = nullptr;  // fragment-major, [Np/32][Kp/32][1024]
    float *d_s = nullptr;   // [N]
    int64_t N = 0, K = 0, Np = 0, Kp = 0;
    bool inf_scale = false;  // some scale is +-inf: enchip_matmul_bt_q8 declines (see there)
};

thread_local std::string g_open_error = "no error";

// The last failure this thread saw on a context (by its id), so that a thread reading
// enchip_last_error after its own failure gets its own message even when another
// thread has failed on the same context since.
struct ThreadError {
    uint64_t ctx_id = 0;
    std::string msg;
};
thread_local ThreadError g_thread_error;
std::atomic<uint64_t> g_next_ctx_id{1};

// Scratch of enchip_w8a8_linear_noalloc_dev: the quantized activations (at most
// kNoAllocCodeBytes) followed by their per-row scales (at most kNoAllocRows floats). One
// copy per device, held for the life of the process, shared by every call on that device.
constexpr size_t kNoAllocCodeBytes = (size_t)32 << 20;
constexpr int64_t kNoAllocRows = (int64_t)1 << 18;
constexpr size_t kNoAllocBytes = kNoAllocCodeBytes + (size_t)kNoAllocRows * sizeof(float);
static __device__ __align__(256) int8_t scratch[kNoAllocBytes];

// Per device: the device address of `scratch` (hipGetSymbolAddress with that device
// current; in host code the name `scratch` is only a stand-in, so kernels and copies get
// this address) and an event recorded after the last call that used it. Every context on
// the device shares both; g_noalloc_mu guards them and is held across a call's whole
// enqueue, so calls from different threads or contexts order themselves through the event.
constexpr int kMaxDevices = 64;
struct NoallocDevice {
    int8_t *ptr = nullptr;
    hipEvent_t ev = nullptr;  // held for the life of the process, like the array
    bool pending = false;     // ev has been recorded since the last capture-free call
};
std::mutex g_noalloc_mu;
NoallocDevice g_noalloc[kMaxDevices];

// Called by enchip_open with `device` current. On failure the no-alloc entry point
// declines on this device; everything else works.
hipError_t noalloc_scratch_init(int device, int8_t **out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(g_noalloc_mu);
    NoallocDevice &d = g_noalloc[device];
    if (!d.ev) {
        hipError_t e = hipEventCreateWithFlags(&d.ev, hipEventDisableTiming);
        if (e != hipSuccess) {
            d.ev = nullptr;
            (void)hipGetLastError();
            return e;
        }
    }
    if (!d.ptr) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return e;
        }
        d.ptr = static_cast<int8_t *>(p);
    }
    *out = d.ptr;
    return hipSuccess;
}

}  // namespace

struct enchip_ctx {
    uint64_t id = 0;  // unique per context for the life of the process
    int device = 0;
    hipStream_t stream = nullptr;
    int num_cus = 0, clock_khz = 0;
    std::string arch;
    std::mutex mu;
    std::string err = "no error";
    int8_t *noalloc = nullptr;  // this device's address of `scratch` (NULL: unavailable)
    std::string noalloc_err;
    std::unordered_map<uint64_t, Weight> weights;
    // Attention kernels whose dynamic-LDS limit has been raised on this context's device
    // (hipFuncSetAttribute, once per kernel and byte count rather than once per launch).
    std::vector<std::pair<const void *, size_t>> lds_set;
    uint64_t next_handle = 1;
    int64_t small_m = 32;
    int att_products = ENCHIP_ATT_FLASH_F16;  // enchip_set_attention_products
    // Device scratch (grown on demand, freed by enchip_close). Each growable buffer is
    // capped at scratch_limit bytes (enchip_set_scratch_limit; 0 = no cap).
    size_t scratch_limit = 0;
    // The last stream that enqueued work on the shared scratch (d_aq, d_as, d_cand) and
    // an event recorded after that work: a user on another stream waits for it first.
    hipEvent_t scratch_ev = nullptr;
    hipStream_t scratch_stream = nullptr;
    bool scratch_pending = false;
    int8_t *d_aq = nullptr;
    size_t aq_cap = 0;
    float *d_as = nullptr;
    size_t as_cap = 0;
    float *d_a = nullptr;
    size_t a_cap = 0;
    float *d_dst = nullptr;
    size_t dst_cap = 0;
    float *d_bias = nullptr;
    size_t bias_cap = 0;
    int32_t *d_acc = nullptr;
    size_t acc_cap = 0;
    float *d_fb = nullptr;  // enchip_matmul_bt_f32's b operand
    size_t fb_cap = 0;
    uint64_t *d_cand = nullptr;  // top-k candidates
    size_t cand_cap = 0;
    // enchip_ann_topk's device results, one block so that one copy brings them back:
    // hit indices (int32, M k), hit scores (f32, M k), then the fused route's list sizes
    // (uint32, M)
    int32_t *d_hits = nullptr;
    size_t hits_cap = 0;
    // enchip_ann_topk routing (enchip_ann_topk_stats)
    int64_t ann_fused_calls = 0, ann_fallbacks = 0;
    // Pinned host staging for the host entry points' large copies (upload / download):
    // two slots of kStageChunk bytes, each fenced by an event recorded after its DMA.
    char *h_stage = nullptr;
    hipEvent_t stage_ev[2] = {nullptr, nullptr};
};

namespace {

int fail(enchip_ctx *c, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    c->err = buf;
    g_thread_error.ctx_id = c->id;
    g_thread_error.msg = buf;
    return code;
}

#define HIP_TRY(ctx, expr)                                                                  \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return fail((ctx), ENCHIP_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

// Grows a device buffer to at least `bytes`. Contents are not preserved. Scratch
// buffers (not weights) are refused past the context's scratch limit, as a failed
// allocation would be.
template <typename T>
int ensure(enchip_ctx *c, T **p, size_t *cap, size_t bytes, bool scratch = true) {
    // checked before the capacity: a call that needs more than the cap declines even
    // when an earlier call already grew the buffer
    if (scratch && c->scratch_limit != 0 && bytes > c->scratch_limit)
        return fail(c, ENCHIP_ERR_OOM, "scratch of %zu bytes exceeds the context's scratch limit of %zu", bytes,
                    c->scratch_limit);
    if (bytes <= *cap && *p) return ENCHIP_OK;
    if (*p) {
        // the old buffer may still be read by work enqueued on another stream
        if (scratch && c->scratch_pending) (void)hipEventSynchronize(c->scratch_ev);
        hipError_t e = hipFree(*p);
        *p = nullptr;
        *cap = 0;
        if (e != hipSuccess) return fail(c, ENCHIP_ERR_HIP, "hipFree: %s", hipGetErrorString(e));
    }
    size_t want = std::max<size_t>(bytes, 256);
    hipError_t e = hipMalloc((void **)p, want);
    if (e != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();
        return fail(c, ENCHIP_ERR_OOM, "hipMalloc(%zu): %s", want, hipGetErrorString(e));
    }
    *cap = want;
    return ENCHIP_OK;
}

int check_launch(enchip_ctx *c, const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(c, ENCHIP_ERR_HIP, "launch %s: %s", what, hipGetErrorString(e));
    return ENCHIP_OK;
}

// A 1-D launch of `blocks` workgroups of `threads` must keep its global thread index
// below 2^32.
bool grid_fits(int64_t blocks, int64_t threads) {
    return blocks >= 0 && blocks * threads < ((int64_t)1 << 32);
}

// Rows per launch of the row kernels (at most 64 threads per row: 2^28 threads).
constexpr int64_t kRowChunk = (int64_t)1 << 22;

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// Host <-> device copies of the host entry points. From pageable memory the runtime moved
// 21-37 GB/s host to device and 16-17 GB/s device to host on MI355X (1.5-24 MB), against
// 43-56 GB/s from pinned memory; a copy into pinned memory followed by the DMA, one after
// the other, gained nothing. So large copies run through two pinned slots of kStageChunk
// bytes: the CPU fills (or empties) one slot while the DMA engine moves the other. Device
// to host from kStageMinDown bytes; host to device, whose pageable rate is better, from
// kStageMinUp (below it the few chunks hide too little of the per-chunk waits).
constexpr size_t kStageChunk = (size_t)1 << 20, kStageMinUp = (size_t)4 << 20, kStageMinDown = (size_t)1 << 20;

int ensure_stage(enchip_ctx *c) {
    if (c->h_stage) return ENCHIP_OK;
    for (hipEvent_t &e : c->stage_ev)
        if (!e) HIP_TRY(c, hipEventCreateWithFlags(&e, hipEventDisableTiming));
    void *p = nullptr;
    hipError_t e = hipHostMalloc(&p, 2 * kStageChunk, hipHostMallocDefault);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(c, ENCHIP_ERR_OOM, "hipHostMalloc(%zu): %s", 2 * kStageChunk, hipGetErrorString(e));
    }
    c->h_stage = static_cast<char *>(p);
    return ENCHIP_OK;
}

// Enqueues the copy of `bytes` from host memory src to device memory dst on s. src may be
// reused once this returns (every byte is in a pinned slot or already on its way).
int upload(enchip_ctx *c, void *dst, const void *src, size_t bytes, hipStream_t s) {
    if (bytes < kStageMinUp) {
        if (bytes) HIP_TRY(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
        return ENCHIP_OK;
    }
    int rc;
    if ((rc = ensure_stage(c))) return rc;
    for (size_t off = 0, i = 0; off < bytes; off += kStageChunk, ++i) {
        const size_t n = std::min(kStageChunk, bytes - off);
        char *slot = c->h_stage + (i & 1) * kStageChunk;
        HIP_TRY(c, hipEventSynchronize(c->stage_ev[i & 1]));  // the slot's last DMA has ended
        std::memcpy(slot, static_cast<const char *>(src) + off, n);
        HIP_TRY(c, hipMemcpyAsync(static_cast<char *>(dst) + off, slot, n, hipMemcpyHostToDevice, s));
        HIP_TRY(c, hipEventRecord(c->stage_ev[i & 1], s));
    }
    return ENCHIP_OK;
}

// Copies `bytes` from device memory src to host memory dst after the work already
// enqueued on s. A small copy is only enqueued (the caller synchronizes s before it reads
// dst); a staged one has completed when this returns.
int download(enchip_ctx *c, void *dst, const void *src, size_t bytes, hipStream_t s) {
    if (bytes < kStageMinDown) {
        if (bytes) HIP_TRY(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
        return ENCHIP_OK;
    }
    int rc;
    if ((rc = ensure_stage(c))) return rc;
    const size_t nch = (bytes + kStageChunk - 1) / kStageChunk;
    auto chunk = [&](size_t i) { return std::min(kStageChunk, bytes - i * kStageChunk); };
    auto enqueue = [&](size_t i) -> int {
        HIP_TRY(c, hipMemcpyAsync(c->h_stage + (i & 1) * kStageChunk, static_cast<const char *>(src) + i * kStageChunk,
                                  chunk(i), hipMemcpyDeviceToHost, s));
        HIP_TRY(c, hipEventRecord(c->stage_ev[i & 1], s));
        return ENCHIP_OK;
    };
    for (hipEvent_t e : c->stage_ev) HIP_TRY(c, hipEventSynchronize(e));  // earlier uploads' DMAs
    if ((rc = enqueue(0))) return rc;
    for (size_t i = 0; i < nch; ++i) {
        // the other slot last held chunk i - 1, already copied out
        if (i + 1 < nch && (rc = enqueue(i + 1))) return rc;
        HIP_TRY(c, hipEventSynchronize(c->stage_ev[i & 1]));
        std::memcpy(static_cast<char *>(dst) + i * kStageChunk, c->h_stage + (i & 1) * kStageChunk, chunk(i));
    }
    return ENCHIP_OK;
}

// Orders work about to use the shared scratch on stream s after the scratch's last
// user on another stream. Under stream capture the caller orders the streams (a
// captured graph cannot wait on an event recorded outside it).
int scratch_wait(enchip_ctx *c, hipStream_t s) {
    if (!c->scratch_pending || c->scratch_stream == s || capturing(s)) return ENCHIP_OK;
    hipError_t e = hipStreamWaitEvent(s, c->scratch_ev, 0);
    if (e != hipSuccess) return fail(c, ENCHIP_ERR_HIP, "hipStreamWaitEvent(scratch): %s", hipGetErrorString(e));
    return ENCHIP_OK;
}

// Marks the scratch as in use by the work just enqueued on stream s.
int scratch_record(enchip_ctx *c, hipStream_t s) {
    if (capturing(s)) return ENCHIP_OK;
    hipError_t e = hipEventRecord(c->scratch_ev, s);
    if (e != hipSuccess) return fail(c, ENCHIP_ERR_HIP, "hipEventRecord(scratch): %s", hipGetErrorString(e));
    c->scratch_stream = s;
    c->scratch_pending = true;
    return ENCHIP_OK;
}

// Quantizes d_a[M,K] into q (zero-padded to ldq) and scale[M]: row-major q[M][ldq], or
// fragment-major (kernels.h frag_off) when frag.
int launch_quant_rows(enchip_ctx *c, const float *d_a, int64_t M, int64_t K, int8_t *q, int64_t ldq,
                      float *scale, hipStream_t s, bool frag);

// Launches in chunks of kRowChunk rows (a multiple of 32, so a fragment-major chunk
// starts at byte r0 * ldq like a row-major one).
int launch_quant(enchip_ctx *c, const float *d_a, int64_t M, int64_t K, int8_t *q, int64_t ldq,
                 float *scale, hipStream_t s, bool frag = false) {
    for (int64_t r0 = 0; r0 < M; r0 += kRowChunk) {
        int rc = launch_quant_rows(c, d_a + r0 * K, std::min(kRowChunk, M - r0), K, q + r0 * ldq, ldq, scale + r0, s,
                                   frag);
        if (rc) return rc;
    }
    return ENCHIP_OK;
}

int launch_quant_rows(enchip_ctx *c, const float *d_a, int64_t M, int64_t K, int8_t *q, int64_t ldq,
                      float *scale, hipStream_t s, bool frag) {
    if (M == 0) return ENCHIP_OK;
    const bool vec = (K % 4 == 0) && (ldq % 4 == 0) && ((uintptr_t)d_a % 16 == 0) &&
                     ((uintptr_t)q % (frag ? 16 : 4) == 0) && K > 0 && (frag ? ldq : K) <= 256 * 16;
    if (vec) {
        const int ch = (int)(((frag ? ldq : K) + 255) / 256);
        const int k = (int)K;
        // fragment-major: 8 rows per block, 2 per wavefront for rows up to 512 floats, else
        // 1 (measured at K = 768 on MI355X: 26.0 -> 24.5 us per 32768 rows with 1 row per
        // wavefront, once every row load was in flight at once)
        const int rpw = ch <= 2 ? 2 : 1;
        const dim3 grid((unsigned)(frag ? (M + 7) / 8 : (M + 3) / 4)), block(frag ? 512 / rpw : 256);
        switch (ch) {
#define QCASE(N)                                                                                                  \
    case N:                                                                                                       \
        if (frag && rpw == 2)                                                                                     \
            hipLaunchKernelGGL((enchip::quant_rows_frag<N, 2>), grid, block, 0, s, d_a, q, ldq, scale, M, k);     \
        else if (frag)                                                                                            \
            hipLaunchKernelGGL((enchip::quant_rows_frag<N, 1>), grid, block, 0, s, d_a, q, ldq, scale, M, k);     \
        else                                                                                                      \
            hipLaunchKernelGGL(enchip::quant_rows_vec<N>, grid, block, 0, s, d_a, q, ldq, scale, M, k);           \
        break;
            QCASE(1) QCASE(2) QCASE(3) QCASE(4) QCASE(5) QCASE(6) QCASE(7) QCASE(8)
            QCASE(9) QCASE(10) QCASE(11) QCASE(12) QCASE(13) QCASE(14) QCASE(15) QCASE(16)
#undef QCASE
            default: return fail(c, ENCHIP_ERR_ARG, "quant: bad chunk count %d", ch);
        }
    } else {
        const dim3 grid((unsigned)((M + 3) / 4)), block(256);
        if (frag)
            hipLaunchKernelGGL(enchip::quant_rows_scalar<true>, grid, block, 0, s, d_a, q, ldq, scale, M, K);
        else
            hipLaunchKernelGGL(enchip::quant_rows_scalar<false>, grid, block, 0, s, d_a, q, ldq, scale, M, K);
    }
    return check_launch(c, "quant_rows");
}

template <int BM, int BN, int EPI, int MINB>
void launch_gemm_t(const Weight &w, const int8_t *aq, int64_t lda, const float *as, const float *bias,
                   void *out, int64_t ldo, int64_t M, hipStream_t s) {
    const int tilesM = (int)((M + BM - 1) / BM), tilesN = (int)((w.N + BN - 1) / BN);
    hipLaunchKernelGGL((enchip::gemm_w8a8<BM, BN, EPI, MINB>), dim3((unsigned)(tilesM * tilesN)), dim3(256), 0,
                       s, aq, lda, w.d_w, as, w.d_s, bias, out, ldo, (int)M, (int)w.N, (int)w.Kp, tilesN);
}

// Tile choice for gemm_w8a8 (the general kernel): 128x256 tiles (2 blocks per CU)
// when they give every CU at least two blocks, otherwise 128x128 tiles (3 blocks per
// CU) to fill the chip.
bool use_wide_tile(const enchip_ctx *c, const Weight &w, int64_t M) {
    const int64_t t256 = ((M + 127) / 128) * ((w.N + 255) / 256);
    return t256 >= 2 * (int64_t)c->num_cus;
}

// Ring depth of gemm_w8a8_pt: 2 stages, so the 64-deep K stages must be even (0 = not
// usable). A 3-stage ring speeds up the bare main loop by 2-9% on MI355X, but with the
// epilogue its register pressure spills and the whole kernel is no faster.
int pt_ring(const Weight &w) {
    return (w.Kp / enchip::PT_BK) % enchip::PT_PW == 0 ? enchip::PT_PW : 0;
}

// gemm_w8a8_pt's preconditions (gemm_persistent.h): a usable ring depth, 16-byte
// aligned A, 32-bit byte offsets into A and the weights, and 16-byte row-major output
// stores (N and the output pitch multiples of 4). Fragment-major A (af) has pitch Kp
// and is read up to the next multiple of PT_BM rows.
bool use_persistent(const Weight &w, const void *aq, int64_t lda, const void *out, int64_t ldo, int64_t M,
                    bool af) {
    const int64_t lim = (int64_t)1 << 31;
    const int64_t a_end = af ? round_up(M, enchip::PT_BM) * w.Kp : (M - 1) * lda + w.Kp;
    return pt_ring(w) != 0 && (lda % 16) == 0 && (!af || lda == w.Kp) && ((uintptr_t)aq % 16) == 0 &&
           a_end < lim && w.Np * w.Kp < lim && (w.N % 4) == 0 && (ldo % 4) == 0 && ((uintptr_t)out % 16) == 0;
}

// True when a GEMM on activations this library quantizes itself (into the context
// scratch, pitch Kp) runs gemm_w8a8_pt, which then takes them fragment-major.
bool route_af(const enchip_ctx *c, const Weight &w, int64_t M, const void *out, int64_t ldo) {
    return M > c->small_m && use_persistent(w, nullptr, w.Kp, out, ldo, M, true);
}

// Small-M kernel choice: gemv_w8a8_wide (one wavefront per 32-channel group, whole K)
// once there are enough groups to spread over the SIMDs, else gemv_w8a8 (one workgroup
// per group, K split over its waves). Measured crossover on MI355X (M=1..16): with
// K <= 1024 the wide kernel is 1.5x faster from 4 groups per CU (N=32768, K=384..768);
// with K=3072 it loses at 2 groups per CU (each wave then walks 96 fragments in series)
// and wins by 1.3x from 8 per CU.
bool gemv_wide(const enchip_ctx *c, const Weight &w) {
    const int64_t groups = (w.N + 31) / 32, cus = c->num_cus;
    return groups >= 8 * cus || (groups >= 4 * cus && w.Kp <= 1024);
}

int persistent_grid(const enchip_ctx *c, int64_t tiles, int per_cu = 2) {
    const int64_t full = std::max<int64_t>(8, ((int64_t)per_cu * c->num_cus) / 8 * 8);
    return (int)std::min<int64_t>(full, (tiles + 7) / 8 * 8);
}

// Tile height of gemm_w8a8_pt for M rows of a weight: 64-row tiles at 3 workgroups per CU
// when 128-row tiles would not fill the 2 per CU slots (small M), else 128. Measured on
// MI355X (K = 768, N = 3072, GELU): M = 4096 46 -> 35 us on config 2's pre-activations and
// 29 -> 25 us on an encoder's; at M = 32768 the 128-row tiles stay faster (164 against 166).
int pt_bm(const enchip_ctx *c, const Weight &w, int64_t M) {
    const int64_t tiles128 = ((M + enchip::PT_BM - 1) / enchip::PT_BM) * ((w.N + enchip::PT_BN - 1) / enchip::PT_BN);
    return tiles128 < 2 * (int64_t)c->num_cus ? enchip::PT_BM_SMALL : enchip::PT_BM;
}

// Main-loop wave priority of gemm_w8a8_pt for a weight and epilogue: raised for the
// bias-only epilogue when N or the padded K is at least 1024. Measured on MI355X (same
// process, interleaved): BERT-base QKV and FFN-down 4-10% faster, XLM-R-large QKV, O and
// FFN-down 6-9% faster; BERT-base O (768 x 768) 4% slower, so it keeps 0. The GELU
// epilogue keeps 0: raised, BERT-base FFN-up took 206 us per launch in the encode against
// 189 us (it ran 3-5% faster on uniformly random codes, whose pre-activations differ).
int pt_prio(const Weight &w, int epi) {
    return (epi == enchip::EPI_F32 || epi == enchip::EPI_TOPK) && (w.N >= 1024 || w.Kp >= 1024) ? 1 : 0;
}

template <int BM, int PW, int EPI, bool AF>
void launch_pt_bm(enchip_ctx *c, const Weight &w, const int8_t *aq, int64_t lda, const float *as, const float *bias,
                  void *out, int64_t ldo, int64_t M, hipStream_t s, const enchip::TopkSink &sink) {
    using namespace enchip;
    const int tilesM = (int)((M + BM - 1) / BM), tilesN = (int)((w.N + PT_BN - 1) / PT_BN);
    const int64_t tiles = (int64_t)tilesM * tilesN;
    const int grid = persistent_grid(c, tiles, BM == PT_BM_SMALL ? 3 : 2);
    if (pt_prio(w, EPI))
        hipLaunchKernelGGL((gemm_w8a8_pt<BM, PT_BN, PT_BK, PW, EPI, AF, PT_NW, 1>), dim3(grid), dim3(64 * PT_NW), 0, s, aq,
                           lda, w.d_w, as, w.d_s, bias, out, ldo, (int)M, (int)w.N, (int)w.Kp, tilesN, (int)tiles, sink);
    else
        hipLaunchKernelGGL((gemm_w8a8_pt<BM, PT_BN, PT_BK, PW, EPI, AF, PT_NW, 0>), dim3(grid), dim3(64 * PT_NW), 0, s, aq,
                           lda, w.d_w, as, w.d_s, bias, out, ldo, (int)M, (int)w.N, (int)w.Kp, tilesN, (int)tiles, sink);
}

template <int PW, int EPI, bool AF>
void launch_pt(enchip_ctx *c, const Weight &w, const int8_t *aq, int64_t lda, const float *as, const float *bias,
               void *out, int64_t ldo, int64_t M, hipStream_t s, const enchip::TopkSink &sink = {}) {
    if (pt_bm(c, w, M) == enchip::PT_BM_SMALL)
        launch_pt_bm<enchip::PT_BM_SMALL, PW, EPI, AF>(c, w, aq, lda, as, bias, out, ldo, M, s, sink);
    else
        launch_pt_bm<enchip::PT_BM, PW, EPI, AF>(c, w, aq, lda, as, bias, out, ldo, M, s, sink);
}

// gemm_w8a8_skinny's shapes (gemm_skinny.h), by Kp / 32 (0: not this kernel): more rows
// than the small-M kernels take and at most 256 (all of them in LDS), Kp / 32 one of 4, 8,
// 12, 16, and at least 1024 groups of 32 channels (N >= 32768: ann indexes). Row-major A
// needs 16-byte aligned rows.
int skinny_shape_nk(const Weight &w, const void *aq, int64_t lda, bool af) {
    const int nk = (int)(w.Kp / 32);
    if ((nk != 4 && nk != 8 && nk != 12 && nk != 16) || (w.N + 31) / 32 < 1024) return 0;
    if (!af && (lda % 16 != 0 || (uintptr_t)aq % 16 != 0 || lda < w.Kp)) return 0;
    return nk;
}

int skinny_nk(const enchip_ctx *c, const Weight &w, int64_t M, const void *aq, int64_t lda, bool af) {
    return M > c->small_m && M <= 256 ? skinny_shape_nk(w, aq, lda, af) : 0;
}

template <int MB, int EPI, bool AF>
void launch_skinny_mb(enchip_ctx *c, const Weight &w, int nk, const int8_t *aq, int64_t lda, const float *as,
                      const float *bias, float *out, int64_t ldo, int64_t M, hipStream_t s,
                      const enchip::TopkSink &sink) {
    using namespace enchip;
    const int64_t groups = (w.N + 31) / 32;
    const dim3 grid((unsigned)std::min<int64_t>(c->num_cus, (groups + SK_WAVES - 1) / SK_WAVES)), block(64 * SK_WAVES);
#define SK_CASE(NK)                                                                                                    \
    case NK:                                                                                                           \
        hipLaunchKernelGGL((gemm_w8a8_skinny<MB, NK, EPI, AF>), grid, block, 0, s, aq, lda, w.d_w, as, w.d_s, bias, \
                           out, ldo, (int)M, (int)w.N, sink);                                                          \
        break;
    switch (nk) {
        SK_CASE(4)
        SK_CASE(8)
        SK_CASE(12)
        SK_CASE(16)
        default: break;
    }
#undef SK_CASE
}

// nk from skinny_nk; 32 x 4 or 32 x 8 rows staged.
template <int EPI, bool AF>
void launch_skinny(enchip_ctx *c, const Weight &w, int nk, const int8_t *aq, int64_t lda, const float *as,
                   const float *bias, float *out, int64_t ldo, int64_t M, hipStream_t s,
                   const enchip::TopkSink &sink = {}) {
    if (M <= 128) launch_skinny_mb<4, EPI, AF>(c, w, nk, aq, lda, as, bias, out, ldo, M, s, sink);
    else launch_skinny_mb<8, EPI, AF>(c, w, nk, aq, lda, as, bias, out, ldo, M, s, sink);
}

// af: aq is fragment-major (the caller checked route_af); otherwise row-major at pitch lda.
// Returns false, launching nothing, when the chosen kernel's grid would not fit.
template <int EPI>
bool launch_gemm_epi(enchip_ctx *c, const Weight &w, const int8_t *aq, int64_t lda, const float *as,
                     const float *bias, void *out, int64_t ldo, int64_t M, hipStream_t s, bool af) {
    if (EPI == enchip::EPI_F32) {
        if (const int nk = skinny_nk(c, w, M, aq, lda, af)) {
            if (af) launch_skinny<enchip::EPI_F32, true>(c, w, nk, aq, lda, as, bias, (float *)out, ldo, M, s);
            else launch_skinny<enchip::EPI_F32, false>(c, w, nk, aq, lda, as, bias, (float *)out, ldo, M, s);
            return true;
        }
    }
    if (af || (M > c->small_m && use_persistent(w, aq, lda, out, ldo, M, false))) {
        if (af) launch_pt<enchip::PT_PW, EPI, true>(c, w, aq, lda, as, bias, out, ldo, M, s);
        else launch_pt<enchip::PT_PW, EPI, false>(c, w, aq, lda, as, bias, out, ldo, M, s);
        return true;
    }
    if (M <= c->small_m) {
        if (gemv_wide(c, w)) {
            const int64_t blocks = (w.N + 32 * enchip::GVW_WAVES - 1) / (32 * enchip::GVW_WAVES);
            if (!grid_fits(blocks, 64 * enchip::GVW_WAVES)) return false;
            hipLaunchKernelGGL((enchip::gemv_w8a8_wide<EPI>), dim3((unsigned)blocks), dim3(64 * enchip::GVW_WAVES), 0,
                               s, aq, lda, w.d_w, as, w.d_s, bias, out, ldo, (int)M, (int)w.N, (int)w.Kp);
        } else {
            const int64_t blocks = (w.N + 31) / 32;
            if (!grid_fits(blocks, 64 * enchip::GV_WAVES) || M > 32) return false;
            // weight fragments per wave and batch: the whole K in one batch up to 32 fragments
            const int64_t per_wave = (w.Kp / 32 + enchip::GV_WAVES - 1) / enchip::GV_WAVES;
            const dim3 grid((unsigned)blocks, (unsigned)((M + enchip::GV_ROWS - 1) / enchip::GV_ROWS));
#define GV_LAUNCH(NB)                                                                                             \
    hipLaunchKernelGGL((enchip::gemv_w8a8<EPI, NB>), grid, dim3(64 * enchip::GV_WAVES), 0, s, aq, lda, w.d_w, as, \
                       w.d_s, bias, out, ldo, (int)M, (int)w.N, (int)w.Kp)
            if (per_wave <= 1) GV_LAUNCH(1);
            else if (per_wave == 2) GV_LAUNCH(2);
            else if (per_wave == 3) GV_LAUNCH(3);
            else if (per_wave == 4) GV_LAUNCH(4);
            else GV_LAUNCH(8);
#undef GV_LAUNCH
        }
        return true;
    }
    const bool wide = use_wide_tile(c, w, M);
    const int64_t tiles = ((M + 127) / 128) * ((w.N + (wide ? 255 : 127)) / (wide ? 256 : 128));
    if (!grid_fits(tiles, 256)) return false;
    if (wide)
        launch_gemm_t<128, 256, EPI, 2>(w, aq, lda, as, bias, out, ldo, M, s);
    else
        launch_gemm_t<128, 128, EPI, 3>(w, aq, lda, as, bias, out, ldo, M, s);
    return true;
}

int launch_gemm(enchip_ctx *c, const Weight &w, const int8_t *aq, int64_t lda, const float *as,
                const float *bias, int epi, void *out, int64_t ldo, int64_t M, hipStream_t s, bool af = false) {
    if (M == 0) return ENCHIP_OK;
    bool ok;
    switch (epi) {
        case enchip::EPI_I32: ok = launch_gemm_epi<enchip::EPI_I32>(c, w, aq, lda, as, bias, out, ldo, M, s, af); break;
        case enchip::EPI_F32: ok = launch_gemm_epi<enchip::EPI_F32>(c, w, aq, lda, as, bias, out, ldo, M, s, af); break;
        case enchip::EPI_F32_GELU:
            ok = launch_gemm_epi<enchip::EPI_F32_GELU>(c, w, aq, lda, as, bias, out, ldo, M, s, af);
            break;
        default: return fail(c, ENCHIP_ERR_ARG, "bad epilogue %d", epi);
    }
    if (!ok)
        return fail(c, ENCHIP_ERR_ARG, "gemm: M=%lld N=%lld needs more workgroups than one launch addresses",
                    (long long)M, (long long)w.N);
    return check_launch(c, "gemm_w8a8");
}

// Weight fragments per wave and batch of gemv_w8a8 (the instantiated 1, 2, 3, 4, 8).
int gv_nb(const Weight &w) {
    const int64_t per_wave = (w.Kp / 32 + enchip::GV_WAVES - 1) / enchip::GV_WAVES;
    return per_wave <= 4 ? (int)std::max<int64_t>(per_wave, 1) : 8;
}

// True when a linear that quantizes its own activations (d_a [M][K] f32, pitch K) runs
// as the single small-M launch gemv_w8a8_q: M within the small-M limit (at most 32, one
// MFMA tile of rows), a narrow N (the wide kernel's streaming form serves wide N), and
// whole float4 rows that fit one wavefront's registers.
bool fused_small_m(const enchip_ctx *c, const Weight &w, int64_t M, const float *d_a) {
    return M >= 1 && M <= c->small_m && M <= 32 && !gemv_wide(c, w) && w.K % 4 == 0 && w.K > 0 &&
           w.K <= enchip::GVQ_MAX_K && (d_a == nullptr || (uintptr_t)d_a % 16 == 0);
}

// float4 per lane that hold one row of K floats in gemv_w8a8_q (K <= 256 * QCH), one of
// the instantiated 1, 2, 3, 4, 8, 12, 16.
int gvq_qch(int64_t K) {
    return K <= 256 ? 1 : K <= 512 ? 2 : K <= 768 ? 3 : K <= 1024 ? 4 : K <= 2048 ? 8 : K <= 3072 ? 12 : 16;
}

// The kernels of gemv_w8a8_q whose dynamic-LDS limit has been raised (process-wide: the
// attribute belongs to the kernel on the current device).
int launch_fused_small_m(enchip_ctx *c, const Weight &w, const float *d_a, int64_t M, const float *bias, int epi,
                         float *out, int64_t ldo, hipStream_t s) {
    using Kern = void (*)(const float *, const int8_t *, const float *, const float *, void *, int64_t, int, int, int, int);
#define GVQ_ROW(E)                                                                                           \
    {enchip::gemv_w8a8_q<E, 1>, enchip::gemv_w8a8_q<E, 2>, enchip::gemv_w8a8_q<E, 3>, enchip::gemv_w8a8_q<E, 4>, \
     enchip::gemv_w8a8_q<E, 8>, enchip::gemv_w8a8_q<E, 12>, enchip::gemv_w8a8_q<E, 16>}
    static constexpr Kern table[2][7] = {GVQ_ROW(enchip::EPI_F32), GVQ_ROW(enchip::EPI_F32_GELU)};
#undef GVQ_ROW
    if (M < 1 || M > 32 || w.K > enchip::GVQ_MAX_K || w.K % 4 != 0)
        return fail(c, ENCHIP_ERR_ARG, "gemv_w8a8_q: M=%lld K=%lld outside its shapes", (long long)M, (long long)w.K);
    const int qch = gvq_qch(w.K);
    const Kern fn = table[epi == enchip::EPI_F32_GELU ? 1 : 0][qch <= 4 ? qch - 1 : qch == 8 ? 4 : qch == 12 ? 5 : 6];
    const size_t lds = (size_t)enchip::gvq_lds_bytes((int)w.Kp);
    if (lds > 64 * 1024) {
        const std::pair<const void *, size_t> key(reinterpret_cast<const void *>(fn), lds);
        if (std::find(c->lds_set.begin(), c->lds_set.end(), key) == c->lds_set.end()) {
            HIP_TRY(c, hipFuncSetAttribute(key.first, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            c->lds_set.push_back(key);
        }
    }
    const dim3 grid((unsigned)((w.N + 31) / 32), (unsigned)((M + enchip::GVQ_ROWS - 1) / enchip::GVQ_ROWS));
    hipLaunchKernelGGL(fn, grid, dim3(64 * enchip::GVQ_WAVES), lds, s, d_a, w.d_w, w.d_s, bias, out, ldo, (int)M,
                       (int)w.N, (int)w.K, (int)w.Kp);
    return check_launch(c, "gemv_w8a8_q");
}

int find_weight(enchip_ctx *c, enchip_weight h, Weight **out) {
    auto it = c->weights.find(h);
    if (it == c->weights.end()) return fail(c, ENCHIP_ERR_HANDLE, "unknown weight handle %llu", (unsigned long long)h);
    *out = &it->second;
    return ENCHIP_OK;
}

// Scratch for the quantized activations of M rows at pitch Kp.
int ensure_act_scratch(enchip_ctx *c, int64_t M, int64_t Kp) {
    const int64_t Mp = round_up(std::max<int64_t>(M, 1), kRowPad);
    int rc = ensure(c, &c->d_aq, &c->aq_cap, (size_t)(Mp * Kp));
    if (rc) return rc;
    return ensure(c, &c->d_as, &c->as_cap, (size_t)Mp * sizeof(float));
}

int act_code(int act) {
    return act == ENCHIP_ACT_GELU ? enchip::EPI_F32_GELU : enchip::EPI_F32;
}

}  // namespace

extern "C" {

int enchip_abi_version(void) { return ENCHIP_ABI_VERSION; }

const char *enchip_last_error(const enchip_ctx *ctx) {
    if (!ctx) return g_open_error.c_str();
    // This thread's own last failure on ctx when it has one; otherwise a copy of the
    // context's latest message taken under its lock. Either way the text is owned by
    // the calling thread (another thread's failure cannot replace it) and stays valid
    // until this thread's next enchip_last_error call.
    thread_local std::string copy;
    if (g_thread_error.ctx_id == ctx->id) {
        copy = g_thread_error.msg;
    } else {
        std::lock_guard<std::mutex> g(const_cast<enchip_ctx *>(ctx)->mu);
        copy = ctx->err;
    }
    return copy.c_str();
}

int enchip_open(int device, enchip_ctx **out) {
    if (!out) {
        g_open_error = "enchip_open: out is NULL";
        return ENCHIP_ERR_ARG;
    }
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        g_open_error = std::string("enchip_open: no HIP device (") + hipGetErrorString(e) + ")";
        (void)hipGetLastError();
        return ENCHIP_ERR_NO_DEVICE;
    }
    if (device < 0 || device >= n) {
        g_open_error = "enchip_open: device index " + std::to_string(device) + " out of range (have " +
                       std::to_string(n) + ")";
        return ENCHIP_ERR_NO_DEVICE;
    }
    hipDeviceProp_t prop;
    if ((e = hipSetDevice(device)) != hipSuccess || (e = hipGetDeviceProperties(&prop, device)) != hipSuccess) {
        g_open_error = std::string("enchip_open: ") + hipGetErrorString(e);
        return ENCHIP_ERR_HIP;
    }
    auto *c = new enchip_ctx();
    c->id = g_next_ctx_id.fetch_add(1);
    c->device = device;
    c->num_cus = prop.multiProcessorCount;
    c->clock_khz = prop.clockRate;
    c->arch = prop.gcnArchName;
    if ((e = noalloc_scratch_init(device, &c->noalloc)) != hipSuccess)
        c->noalloc_err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
    if ((e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess) {
        g_open_error = std::string("enchip_open: hipStreamCreate: ") + hipGetErrorString(e);
        delete c;
        return ENCHIP_ERR_HIP;
    }
    if ((e = hipEventCreateWithFlags(&c->scratch_ev, hipEventDisableTiming)) != hipSuccess) {
        g_open_error = std::string("enchip_open: hipEventCreate: ") + hipGetErrorString(e);
        (void)hipStreamDestroy(c->stream);
        delete c;
        return ENCHIP_ERR_HIP;
    }
    *out = c;
    return ENCHIP_OK;
}

int enchip_close(enchip_ctx *ctx) {
    if (!ctx) return ENCHIP_OK;
    {
        std::lock_guard<std::mutex> g(ctx->mu);
        (void)hipSetDevice(ctx->device);
        if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
        if (ctx->scratch_pending) (void)hipEventSynchronize(ctx->scratch_ev);
        for (auto &kv : ctx->weights) {
            (void)hipFree(kv.second.d_w);
            (void)hipFree(kv.second.d_s);
        }
        ctx->weights.clear();
        void *bufs[] = {ctx->d_aq,  ctx->d_as, ctx->d_a,     ctx->d_dst,     ctx->d_bias,
                        ctx->d_acc, ctx->d_fb, ctx->d_cand, ctx->d_hits};
        for (void *p : bufs)
            if (p) (void)hipFree(p);
        if (ctx->scratch_ev) (void)hipEventDestroy(ctx->scratch_ev);
        for (hipEvent_t e : ctx->stage_ev)
            if (e) (void)hipEventDestroy(e);
        if (ctx->h_stage) (void)hipHostFree(ctx->h_stage);
        if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    }
    delete ctx;
    return ENCHIP_OK;
}

int enchip_device_info(enchip_ctx *ctx, int *num_cus, int *clock_khz, char *name, int name_len) {
    if (!ctx) return ENCHIP_ERR_ARG;
    if (num_cus) *num_cus = ctx->num_cus;
    if (clock_khz) *clock_khz = ctx->clock_khz;
    if (name && name_len > 0) {
        std::strncpy(name, ctx->arch.c_str(), (size_t)name_len - 1);
        name[name_len - 1] = 0;
    }
    return ENCHIP_OK;
}

int enchip_gemm_kernel_name(enchip_ctx *ctx, enchip_weight h, int64_t M, int act, char *buf, int len) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if (!buf || len <= 0) return fail(ctx, ENCHIP_ERR_ARG, "gemm_kernel_name: bad buffer");
    const int epi = act_code(act);
    char name[96];
    const int sk = epi == enchip::EPI_F32 ? skinny_nk(ctx, *w, M, nullptr, w->Kp, true) : 0;
    if (sk)  // the library's own quantization is fragment-major (pre_dev's row-major codes: false)
        snprintf(name, sizeof name, "enchip::gemm_w8a8_skinny<%d, %d, %d, true>", M <= 128 ? 4 : 8, sk, epi);
    else if (route_af(ctx, *w, M, nullptr, w->N))
        snprintf(name, sizeof name, "enchip::gemm_w8a8_pt<%d, %d, %d, %d, %d, true, %d, %d>", pt_bm(ctx, *w, M),
                 enchip::PT_BN, enchip::PT_BK, pt_ring(*w), epi, enchip::PT_NW, pt_prio(*w, epi));
    else if (fused_small_m(ctx, *w, M, nullptr) && epi != enchip::EPI_I32)
        snprintf(name, sizeof name, "enchip::gemv_w8a8_q<%d, %d>", epi, gvq_qch(w->K));
    else if (M <= ctx->small_m && gemv_wide(ctx, *w))
        snprintf(name, sizeof name, "enchip::gemv_w8a8_wide<%d>", epi);
    else if (M <= ctx->small_m)
        snprintf(name, sizeof name, "enchip::gemv_w8a8<%d, %d>", epi, gv_nb(*w));
    else if (use_persistent(*w, nullptr, w->Kp, nullptr, w->N, M, false))
        snprintf(name, sizeof name, "enchip::gemm_w8a8_pt<%d, %d, %d, %d, %d, false, %d, %d>", pt_bm(ctx, *w, M),
                 enchip::PT_BN, enchip::PT_BK, pt_ring(*w), epi, enchip::PT_NW, pt_prio(*w, epi));
    else if (use_wide_tile(ctx, *w, M))
        snprintf(name, sizeof name, "enchip::gemm_w8a8<128, 256, %d, 2>", epi);
    else
        snprintf(name, sizeof name, "enchip::gemm_w8a8<128, 128, %d, 3>", epi);
    std::strncpy(buf, name, (size_t)len - 1);
    buf[len - 1] = 0;
    return ENCHIP_OK;
}

int enchip_probe_ceilings(enchip_ctx *ctx, enchip_ceilings *out) {
    if (!ctx || !out) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    const int64_t bytes = (int64_t)1 << 30;
    void *buf = nullptr;
    int *sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipMalloc(&buf, (size_t)bytes);
    if (e != hipSuccess) return fail(ctx, ENCHIP_ERR_OOM, "probe: hipMalloc(1 GiB): %s", hipGetErrorString(e));
    int rc = ENCHIP_OK;
    auto best_us = [&](auto launch, float *best) -> hipError_t {
        hipError_t err;
        *best = 1e30f;
        for (int rep = 0; rep < 6; ++rep) {
            if ((err = hipEventRecord(e0, ctx->stream)) != hipSuccess) return err;
            launch();
            if ((err = hipGetLastError()) != hipSuccess) return err;
            if ((err = hipEventRecord(e1, ctx->stream)) != hipSuccess) return err;
            if ((err = hipEventSynchronize(e1)) != hipSuccess) return err;
            float ms = 0;
            if ((err = hipEventElapsedTime(&ms, e0, e1)) != hipSuccess) return err;
            if (rep > 0 && ms * 1e3f < *best) *best = ms * 1e3f;  // rep 0 is warm-up
        }
        return hipSuccess;
    };
    do {
        if ((e = hipMalloc((void **)&sink, 1 << 20)) != hipSuccess) break;
        if ((e = hipEventCreate(&e0)) != hipSuccess || (e = hipEventCreate(&e1)) != hipSuccess) break;
        if ((e = hipMemsetAsync(buf, 0x11, (size_t)bytes, ctx->stream)) != hipSuccess) break;
        const int64_t n16 = bytes / 16;
        const unsigned grid = (unsigned)(ctx->num_cus * 8);
        float us = 0, best = 1e30f;
        // the best of 8 or 16 loads in flight per lane, 8 or 16 blocks per CU
        for (int variant = 0; variant < 4; ++variant) {
            const unsigned vg = (unsigned)(ctx->num_cus * (variant & 1 ? 16 : 8));
            if ((e = best_us([&] {
                     if (variant < 2)
                         hipLaunchKernelGGL(enchip::probe_stream_read<8>, dim3(vg), dim3(256), 0, ctx->stream,
                                            (const enchip::i32x4_p *)buf, n16, sink);
                     else
                         hipLaunchKernelGGL(enchip::probe_stream_read<16>, dim3(vg), dim3(256), 0, ctx->stream,
                                            (const enchip::i32x4_p *)buf, n16, sink);
                 }, &us)) != hipSuccess) break;
            best = std::min(best, us);
        }
        if (e != hipSuccess) break;
        out->hbm_read_gbps = (double)bytes / best / 1e3;
        if ((e = best_us([&] {
                 hipLaunchKernelGGL(enchip::probe_stream_write, dim3(grid), dim3(256), 0, ctx->stream,
                                    (enchip::i32x4_p *)buf, n16);
             }, &us)) != hipSuccess) break;
        out->hbm_write_gbps = (double)bytes / us / 1e3;
        const int iters = 2000;
        const unsigned mgrid = (unsigned)(ctx->num_cus * 2);
        long long *clk = reinterpret_cast<long long *>(buf);  // the streaming probes are done with buf
        int wall_khz = 0;
        if ((e = hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, ctx->device)) != hipSuccess) break;
        std::vector<long long> ticks(2 * (size_t)mgrid);
        // the mean shader clock (MHz) of the last launch's blocks: s_memtime ticks over
        // s_memrealtime ticks, times the constant clock's rate
        auto clock_mhz = [&](double *mhz) -> hipError_t {
            hipError_t err = hipMemcpyAsync(ticks.data(), clk, ticks.size() * sizeof(long long), hipMemcpyDeviceToHost,
                                            ctx->stream);
            if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
            if (err != hipSuccess) return err;
            double sum = 0;
            int n = 0;
            for (unsigned b = 0; b < mgrid; ++b)
                if (ticks[2 * b + 1] > 0) {
                    sum += (double)ticks[2 * b] / (double)ticks[2 * b + 1];
                    ++n;
                }
            *mhz = n ? sum / n * wall_khz / 1e3 : 0.0;
            return hipSuccess;
        };
        for (int data = 0; data < 2 && e == hipSuccess; ++data) {
            if ((e = best_us([&] {
                     if (data)
                         hipLaunchKernelGGL(enchip::probe_mfma_i8<true>, dim3(mgrid), dim3(256), 0, ctx->stream, sink, iters, clk);
                     else
                         hipLaunchKernelGGL(enchip::probe_mfma_i8<false>, dim3(mgrid), dim3(256), 0, ctx->stream, sink, iters, clk);
                 }, &us)) != hipSuccess) break;
            const double tops = (double)mgrid * 4 * iters * 8 * 65536.0 / us / 1e6;
            double mhz = 0;
            if ((e = clock_mhz(&mhz)) != hipSuccess) break;
            (data ? out->mfma_i8_data_tops : out->mfma_i8_tops) = tops;
            (data ? out->mfma_i8_data_mhz : out->mfma_i8_mhz) = mhz;
        }
        if (e != hipSuccess) break;
        const int viters = 4096;
        const unsigned vgrid = (unsigned)(ctx->num_cus * 8);  // 8 waves per SIMD
        if ((e = best_us([&] {
                 hipLaunchKernelGGL(enchip::probe_valu_f32, dim3(vgrid), dim3(256), 0, ctx->stream,
                                    reinterpret_cast<float *>(buf), viters, 0.999f, 0.5f);
             }, &us)) != hipSuccess) break;
        out->valu_f32_tops = (double)vgrid * 256 * 8 * 2 * viters / us / 1e6;
    } while (0);
    if (e != hipSuccess) rc = fail(ctx, ENCHIP_ERR_HIP, "probe: %s", hipGetErrorString(e));
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (sink) (void)hipFree(sink);
    (void)hipFree(buf);
    return rc;
}

int enchip_set_scratch_limit(enchip_ctx *ctx, int64_t bytes) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (bytes < 0) return fail(ctx, ENCHIP_ERR_ARG, "scratch limit must be >= 0, got %lld", (long long)bytes);
    ctx->scratch_limit = (size_t)bytes;
    return ENCHIP_OK;
}

int enchip_set_small_m(enchip_ctx *ctx, int64_t max_m) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (max_m < 0 || max_m > 32) return fail(ctx, ENCHIP_ERR_ARG, "small_m must be in [0,32], got %lld", (long long)max_m);
    ctx->small_m = max_m;
    return ENCHIP_OK;
}

int enchip_quant_rows_dev(enchip_ctx *ctx, const float *d_a, int64_t M, int64_t K, int8_t *d_aq, int64_t ldq,
                          float *d_ascale, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (M < 0 || K < 0 || K > kMaxK || ldq < K || ldq < 1)
        return fail(ctx, ENCHIP_ERR_ARG, "quant: bad shape M=%lld K=%lld ldq=%lld", (long long)M, (long long)K, (long long)ldq);
    if (M == 0) return ENCHIP_OK;
    if ((K > 0 && !d_a) || !d_aq || !d_ascale) return fail(ctx, ENCHIP_ERR_ARG, "quant: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    return launch_quant(ctx, d_a, M, K, d_aq, ldq, d_ascale, s);
}

int enchip_w8a8_pre_dev(enchip_ctx *ctx, enchip_weight h, const int8_t *d_aq, int64_t ldq, int64_t M,
                        const float *d_ascale, const float *d_bias, int act, float *d_dst, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if (M < 0 || M > ((int64_t)1 << 30)) return fail(ctx, ENCHIP_ERR_ARG, "pre: bad M=%lld", (long long)M);
    if (ldq % 64 != 0 || ldq < w->Kp)
        return fail(ctx, ENCHIP_ERR_ARG, "pre: ldq=%lld must be a multiple of 64 and >= %lld", (long long)ldq, (long long)w->Kp);
    if (act != ENCHIP_ACT_NONE && act != ENCHIP_ACT_GELU) return fail(ctx, ENCHIP_ERR_ARG, "pre: bad act %d", act);
    if (M == 0) return ENCHIP_OK;
    if (!d_aq || !d_ascale || !d_dst) return fail(ctx, ENCHIP_ERR_ARG, "pre: null pointer");
    if ((uintptr_t)d_aq % 16 != 0) return fail(ctx, ENCHIP_ERR_ARG, "pre: d_aq must be 16-byte aligned");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    return launch_gemm(ctx, *w, d_aq, ldq, d_ascale, d_bias, act_code(act), d_dst, w->N, M, s);
}

int enchip_frag_route(enchip_ctx *ctx, enchip_weight h, int64_t M, int64_t *ldq) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return 0;
    if (ldq) *ldq = w->Kp;
    return (M > 0 && M <= ((int64_t)1 << 30) && route_af(ctx, *w, M, nullptr, w->N)) ? 1 : 0;
}

int enchip_quant_rows_frag_dev(enchip_ctx *ctx, const float *d_a, int64_t M, int64_t K, int8_t *d_aq, int64_t ldq,
                               float *d_ascale, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (M < 0 || K < 0 || K > kMaxK || ldq < K || ldq % 64 != 0 || ldq < 64)
        return fail(ctx, ENCHIP_ERR_ARG, "quant_frag: bad shape M=%lld K=%lld ldq=%lld (ldq a multiple of 64 >= K)",
                    (long long)M, (long long)K, (long long)ldq);
    if (M == 0) return ENCHIP_OK;
    if ((K > 0 && !d_a) || !d_aq || !d_ascale) return fail(ctx, ENCHIP_ERR_ARG, "quant_frag: null pointer");
    if ((uintptr_t)d_aq % 16 != 0) return fail(ctx, ENCHIP_ERR_ARG, "quant_frag: d_aq must be 16-byte aligned");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    return launch_quant(ctx, d_a, M, K, d_aq, ldq, d_ascale, s, true);
}

int enchip_quant_rows_frag_gelu_dev(enchip_ctx *ctx, const float *d_a, int64_t M, int64_t K, int8_t *d_aq,
                                    int64_t ldq, float *d_ascale, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (M < 0 || K <= 0 || K % 4 != 0 || ldq < K || ldq % 64 != 0 || ldq > 256 * 16)
        return fail(ctx, ENCHIP_ERR_ARG,
                    "quant_frag_gelu: bad shape M=%lld K=%lld ldq=%lld (K a positive multiple of 4, ldq a multiple of "
                    "64 with K <= ldq <= 4096)",
                    (long long)M, (long long)K, (long long)ldq);
    if (M == 0) return ENCHIP_OK;
    if (!d_a || !d_aq || !d_ascale) return fail(ctx, ENCHIP_ERR_ARG, "quant_frag_gelu: null pointer");
    if ((uintptr_t)d_a % 16 != 0 || (uintptr_t)d_aq % 16 != 0)
        return fail(ctx, ENCHIP_ERR_ARG, "quant_frag_gelu: d_a and d_aq must be 16-byte aligned");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    const int ch = (int)((ldq + 255) / 256), k = (int)K;
    for (int64_t r0 = 0; r0 < M; r0 += kRowChunk) {
        const int64_t rows = std::min(kRowChunk, M - r0);
        const float *a = d_a + r0 * K;
        int8_t *q = d_aq + r0 * ldq;
        float *sc = d_ascale + r0;
        const dim3 grid((unsigned)((rows + 7) / 8)), block(512);
        switch (ch) {
#define QGCASE(N)                                                                                    \
    case N:                                                                                          \
        hipLaunchKernelGGL(enchip::quant_rows_frag_gelu<N>, grid, block, 0, s, a, q, ldq, sc, rows, k); \
        break;
            QGCASE(1) QGCASE(2) QGCASE(3) QGCASE(4) QGCASE(5) QGCASE(6) QGCASE(7) QGCASE(8)
            QGCASE(9) QGCASE(10) QGCASE(11) QGCASE(12) QGCASE(13) QGCASE(14) QGCASE(15) QGCASE(16)
#undef QGCASE
            default: return fail(ctx, ENCHIP_ERR_ARG, "quant_frag_gelu: bad chunk count %d", ch);
        }
        int rc = check_launch(ctx, "quant_rows_frag_gelu");
        if (rc) return rc;
    }
    return ENCHIP_OK;
}

int enchip_w8a8_pre_frag_dev(enchip_ctx *ctx, enchip_weight h, const int8_t *d_aq, int64_t ldq, int64_t M,
                             const float *d_ascale, const float *d_bias, int act, float *d_dst, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if (M < 0 || M > ((int64_t)1 << 30)) return fail(ctx, ENCHIP_ERR_ARG, "pre_frag: bad M=%lld", (long long)M);
    if (ldq != w->Kp)
        return fail(ctx, ENCHIP_ERR_ARG, "pre_frag: ldq=%lld must equal the padded K %lld", (long long)ldq, (long long)w->Kp);
    if (act != ENCHIP_ACT_NONE && act != ENCHIP_ACT_GELU) return fail(ctx, ENCHIP_ERR_ARG, "pre_frag: bad act %d", act);
    if (M == 0) return ENCHIP_OK;
    if (!d_aq || !d_ascale || !d_dst) return fail(ctx, ENCHIP_ERR_ARG, "pre_frag: null pointer");
    if ((uintptr_t)d_aq % 16 != 0) return fail(ctx, ENCHIP_ERR_ARG, "pre_frag: d_aq must be 16-byte aligned");
    if (!route_af(ctx, *w, M, d_dst, w->N))
        return fail(ctx, ENCHIP_ERR_ARG,
                    "pre_frag: M=%lld N=%lld has no fragment-major GEMM route (needs M > %lld, N %% 4 == 0, a "
                    "16-byte aligned d_dst); use enchip_w8a8_pre_dev",
                    (long long)M, (long long)w->N, (long long)ctx->small_m);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    return launch_gemm(ctx, *w, d_aq, ldq, d_ascale, d_bias, act_code(act), d_dst, w->N, M, s, true);
}

int enchip_quant_rows(enchip_ctx *ctx, const float *a, int64_t M, int64_t K, int8_t *aq, float *ascale) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (M < 0 || K < 0 || K > kMaxK) return fail(ctx, ENCHIP_ERR_ARG, "quant: bad shape M=%lld K=%lld", (long long)M, (long long)K);
    if (M == 0) return ENCHIP_OK;
    if (!aq || !ascale || (K > 0 && !a)) return fail(ctx, ENCHIP_ERR_ARG, "quant: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    int rc;
    const int64_t ldq = std::max<int64_t>(K, 1);
    if ((rc = ensure(ctx, &ctx->d_a, &ctx->a_cap, (size_t)(M * K) * sizeof(float)))) return rc;
    if ((rc = ensure(ctx, &ctx->d_aq, &ctx->aq_cap, (size_t)(M * ldq)))) return rc;
    if ((rc = ensure(ctx, &ctx->d_as, &ctx->as_cap, (size_t)M * sizeof(float)))) return rc;
    if ((rc = scratch_wait(ctx, ctx->stream))) return rc;
    if ((rc = upload(ctx, ctx->d_a, a, (size_t)(M * K) * sizeof(float), ctx->stream))) return rc;
    if ((rc = launch_quant(ctx, ctx->d_a, M, K, ctx->d_aq, ldq, ctx->d_as, ctx->stream))) return rc;
    if ((rc = scratch_record(ctx, ctx->stream))) return rc;
    if ((rc = download(ctx, aq, ctx->d_aq, (size_t)(M * K), ctx->stream))) return rc;
    if ((rc = download(ctx, ascale, ctx->d_as, (size_t)M * sizeof(float), ctx->stream))) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return ENCHIP_OK;
}

}  // extern "C"

namespace {

// Copies a fragment-major image (Np * Kp bytes) and the N scales to the device and
// records the weight under a new handle.
int upload_weight(enchip_ctx *ctx, Weight w, const int8_t *image, const float *wscale, enchip_weight *out) {
    int rc;
    size_t wcap = 0, scap = 0;
    const size_t bytes = (size_t)(w.Np * w.Kp);
    for (int64_t n = 0; n < w.N; ++n) w.inf_scale |= std::isinf(wscale[n]);
    if ((rc = ensure(ctx, &w.d_w, &wcap, bytes, false))) return rc;
    if ((rc = ensure(ctx, &w.d_s, &scap, (size_t)w.N * sizeof(float), false))) {
        (void)hipFree(w.d_w);
        return rc;
    }
    hipError_t e1 = hipMemcpy(w.d_w, image, bytes, hipMemcpyHostToDevice);
    hipError_t e2 = hipMemcpy(w.d_s, wscale, (size_t)w.N * sizeof(float), hipMemcpyHostToDevice);
    if (e1 != hipSuccess || e2 != hipSuccess) {
        (void)hipFree(w.d_w);
        (void)hipFree(w.d_s);
        return fail(ctx, ENCHIP_ERR_HIP, "weight upload: %s", hipGetErrorString(e1 != hipSuccess ? e1 : e2));
    }
    const uint64_t h = ctx->next_handle++;
    ctx->weights[h] = w;
    *out = h;
    return ENCHIP_OK;
}

Weight weight_shape(int64_t N, int64_t K) {
    Weight w;
    w.N = N;
    w.K = K;
    w.Np = round_up(N, kColPad);
    w.Kp = round_up(std::max<int64_t>(K, 1), 64);
    return w;
}

}  // namespace

extern "C" {

int64_t enchip_weight_image_bytes(int64_t N, int64_t K) {
    if (N <= 0 || K < 0 || K > kMaxK || N > (int64_t)1 << 30) return -1;
    const Weight w = weight_shape(N, K);
    return w.Np * w.Kp;
}

int enchip_weight_register_image(enchip_ctx *ctx, const int8_t *image, int64_t image_bytes, const float *wscale,
                                 int64_t N, int64_t K, enchip_weight *out) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (!out) return fail(ctx, ENCHIP_ERR_ARG, "weight_register_image: out is NULL");
    *out = 0;
    const int64_t want = enchip_weight_image_bytes(N, K);
    if (want < 0) return fail(ctx, ENCHIP_ERR_ARG, "weight_register_image: bad shape N=%lld K=%lld", (long long)N,
                              (long long)K);
    if (image_bytes != want)
        return fail(ctx, ENCHIP_ERR_ARG, "weight_register_image: image is %lld bytes, N=%lld K=%lld needs %lld",
                    (long long)image_bytes, (long long)N, (long long)K, (long long)want);
    if (!image || !wscale) return fail(ctx, ENCHIP_ERR_ARG, "weight_register_image: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    return upload_weight(ctx, weight_shape(N, K), image, wscale, out);
}

int enchip_weight_export(enchip_ctx *ctx, enchip_weight h, int8_t *image, int64_t image_bytes, float *wscale) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if (image_bytes != w->Np * w->Kp)
        return fail(ctx, ENCHIP_ERR_ARG, "weight_export: buffer is %lld bytes, the image is %lld",
                    (long long)image_bytes, (long long)(w->Np * w->Kp));
    if (!image) return fail(ctx, ENCHIP_ERR_ARG, "weight_export: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    HIP_TRY(ctx, hipMemcpy(image, w->d_w, (size_t)image_bytes, hipMemcpyDeviceToHost));
    if (wscale) HIP_TRY(ctx, hipMemcpy(wscale, w->d_s, (size_t)w->N * sizeof(float), hipMemcpyDeviceToHost));
    return ENCHIP_OK;
}

int enchip_weight_register(enchip_ctx *ctx, const int8_t *wq, const float *wscale, int64_t N, int64_t K,
                           enchip_weight *out) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (!out) return fail(ctx, ENCHIP_ERR_ARG, "weight_register: out is NULL");
    *out = 0;
    if (N <= 0 || K < 0 || K > kMaxK || N > (int64_t)1 << 30)
        return fail(ctx, ENCHIP_ERR_ARG, "weight_register: bad shape N=%lld K=%lld", (long long)N, (long long)K);
    if ((K > 0 && !wq) || !wscale) return fail(ctx, ENCHIP_ERR_ARG, "weight_register: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    const Weight w = weight_shape(N, K);
    // Pre-swizzle on the host into the fragment-major MFMA operand layout.
    const int64_t nk32 = w.Kp / 32;
    std::vector<int8_t> frag((size_t)(w.Np * w.Kp), 0);
    for (int64_t n = 0; n < N; ++n) {
        const int8_t *src = wq + n * K;
        const int64_t nb = n >> 5, nl = n & 31;
        for (int64_t k = 0; k < K; ++k) {
            const int64_t kb = k >> 5, kh = (k >> 4) & 1, j = k & 15;
            frag[(size_t)((nb * nk32 + kb) * 1024 + (nl + 32 * kh) * 16 + j)] = src[k];
        }
    }
    return upload_weight(ctx, w, frag.data(), wscale, out);
}

int enchip_weight_release(enchip_ctx *ctx, enchip_weight h) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    (void)hipFree(w->d_w);
    (void)hipFree(w->d_s);
    ctx->weights.erase(h);
    return ENCHIP_OK;
}

int enchip_weight_shape(enchip_ctx *ctx, enchip_weight h, int64_t *N, int64_t *K) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if (N) *N = w->N;
    if (K) *K = w->K;
    return ENCHIP_OK;
}

int enchip_w8a8_linear_dev(enchip_ctx *ctx, enchip_weight h, const float *d_a, int64_t M, const float *d_bias,
                           int act, float *d_dst, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if (M < 0 || M > ((int64_t)1 << 30)) return fail(ctx, ENCHIP_ERR_ARG, "linear: bad M=%lld", (long long)M);
    if (act != ENCHIP_ACT_NONE && act != ENCHIP_ACT_GELU) return fail(ctx, ENCHIP_ERR_ARG, "linear: bad act %d", act);
    if (M == 0) return ENCHIP_OK;
    if ((w->K > 0 && !d_a) || !d_dst) return fail(ctx, ENCHIP_ERR_ARG, "linear: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    if (fused_small_m(ctx, *w, M, d_a))  // one launch, no scratch
        return launch_fused_small_m(ctx, *w, d_a, M, d_bias, act_code(act), d_dst, w->N, s);
    if ((rc = ensure_act_scratch(ctx, M, w->Kp))) return rc;
    if ((rc = scratch_wait(ctx, s))) return rc;
    const bool af = route_af(ctx, *w, M, d_dst, w->N);
    if ((rc = launch_quant(ctx, d_a, M, w->K, ctx->d_aq, w->Kp, ctx->d_as, s, af))) return rc;
    if ((rc = launch_gemm(ctx, *w, ctx->d_aq, w->Kp, ctx->d_as, d_bias, act_code(act), d_dst, w->N, M, s, af)))
        return rc;
    return scratch_record(ctx, s);
}

int enchip_w8a8_linear_noalloc_dev(enchip_ctx *ctx, enchip_weight h, const float *d_a, int64_t M,
                                   const float *d_bias, int act, float *d_dst, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if (M < 0 || M > kNoAllocRows) return fail(ctx, ENCHIP_ERR_ARG, "linear_noalloc: bad M=%lld (at most %lld rows)",
                                               (long long)M, (long long)kNoAllocRows);
    if (act != ENCHIP_ACT_NONE && act != ENCHIP_ACT_GELU) return fail(ctx, ENCHIP_ERR_ARG, "linear_noalloc: bad act %d", act);
    if (M == 0) return ENCHIP_OK;
    if ((w->K > 0 && !d_a) || !d_dst) return fail(ctx, ENCHIP_ERR_ARG, "linear_noalloc: null pointer");
    if (fused_small_m(ctx, *w, M, d_a)) {  // one launch that quantizes in on-chip memory
        HIP_TRY(ctx, hipSetDevice(ctx->device));
        return launch_fused_small_m(ctx, *w, d_a, M, d_bias, act_code(act), d_dst, w->N,
                                    stream ? (hipStream_t)stream : ctx->stream);
    }
    if (!ctx->noalloc) return fail(ctx, ENCHIP_ERR_HIP, "linear_noalloc: %s", ctx->noalloc_err.c_str());
    // fragment-major codes are read up to the next multiple of PT_BM rows, row-major
    // ones up to row M - 1 (the same routes as enchip_w8a8_linear_dev)
    const bool af = route_af(ctx, *w, M, d_dst, w->N);
    const int64_t code_bytes = (af ? round_up(M, enchip::PT_BM) : M) * w->Kp;
    if ((size_t)code_bytes > kNoAllocCodeBytes)
        return fail(ctx, ENCHIP_ERR_ARG, "linear_noalloc: M=%lld x padded K %lld needs %lld code bytes, more than the "
                    "%zu of the no-alloc scratch", (long long)M, (long long)w->Kp, (long long)code_bytes,
                    kNoAllocCodeBytes);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    int8_t *aq = ctx->noalloc;
    float *as = reinterpret_cast<float *>(ctx->noalloc + kNoAllocCodeBytes);
    // The device's array is shared by every context and stream: this call's quantizer
    // waits for the previous call's GEMM (an event wait, which allocates nothing), and
    // its GEMM records the event for the next. Under stream capture neither happens (a
    // captured graph cannot wait on an event recorded outside it): the caller orders
    // captured calls, and calls that overlap on one GPU then race.
    std::lock_guard<std::mutex> gd(g_noalloc_mu);
    NoallocDevice &nd = g_noalloc[ctx->device];
    const bool cap = capturing(s);
    if (!cap && nd.pending) HIP_TRY(ctx, hipStreamWaitEvent(s, nd.ev, 0));
    // Every code the GEMM reads for rows < M (columns [K, Kp) zero) and every scale is
    // written by the quantizer first, so nothing from an earlier call is read.
    if ((rc = launch_quant(ctx, d_a, M, w->K, aq, w->Kp, as, s, af))) return rc;
    if ((rc = launch_gemm(ctx, *w, aq, w->Kp, as, d_bias, act_code(act), d_dst, w->N, M, s, af))) return rc;
    if (!cap) {
        HIP_TRY(ctx, hipEventRecord(nd.ev, s));
        nd.pending = true;
    }
    return ENCHIP_OK;
}

int enchip_w8a8_linear(enchip_ctx *ctx, enchip_weight h, const float *a, int64_t M, const float *bias, int act,
                       float *dst, int32_t *acc_debug) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if (M < 0 || M > ((int64_t)1 << 30)) return fail(ctx, ENCHIP_ERR_ARG, "linear: bad M=%lld", (long long)M);
    if (act != ENCHIP_ACT_NONE && act != ENCHIP_ACT_GELU) return fail(ctx, ENCHIP_ERR_ARG, "linear: bad act %d", act);
    if (M == 0) return ENCHIP_OK;
    if ((w->K > 0 && !a) || !dst) return fail(ctx, ENCHIP_ERR_ARG, "linear: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    const int64_t K = w->K, N = w->N;
    const size_t out_bytes = (size_t)(M * N) * sizeof(float);
    if ((rc = ensure(ctx, &ctx->d_a, &ctx->a_cap, (size_t)(M * K) * sizeof(float)))) return rc;
    if ((rc = ensure(ctx, &ctx->d_dst, &ctx->dst_cap, out_bytes))) return rc;
    if ((rc = ensure_act_scratch(ctx, M, w->Kp))) return rc;
    if (bias && (rc = ensure(ctx, &ctx->d_bias, &ctx->bias_cap, (size_t)N * sizeof(float)))) return rc;
    if (acc_debug && (rc = ensure(ctx, &ctx->d_acc, &ctx->acc_cap, out_bytes))) return rc;
    hipStream_t s = ctx->stream;
    if ((rc = scratch_wait(ctx, s))) return rc;
    if ((rc = upload(ctx, ctx->d_a, a, (size_t)(M * K) * sizeof(float), s))) return rc;
    if (bias && (rc = upload(ctx, ctx->d_bias, bias, (size_t)N * sizeof(float), s))) return rc;
    const bool af = route_af(ctx, *w, M, ctx->d_dst, N) && (!acc_debug || route_af(ctx, *w, M, ctx->d_acc, N));
    if (!acc_debug && fused_small_m(ctx, *w, M, ctx->d_a)) {
        if ((rc = launch_fused_small_m(ctx, *w, ctx->d_a, M, bias ? ctx->d_bias : nullptr, act_code(act), ctx->d_dst,
                                       N, s)))
            return rc;
    } else {
        if ((rc = launch_quant(ctx, ctx->d_a, M, K, ctx->d_aq, w->Kp, ctx->d_as, s, af))) return rc;
        if ((rc = launch_gemm(ctx, *w, ctx->d_aq, w->Kp, ctx->d_as, bias ? ctx->d_bias : nullptr, act_code(act),
                              ctx->d_dst, N, M, s, af)))
            return rc;
    }
    if (acc_debug &&
        (rc = launch_gemm(ctx, *w, ctx->d_aq, w->Kp, ctx->d_as, nullptr, enchip::EPI_I32, ctx->d_acc, N, M, s, af)))
        return rc;
    if ((rc = scratch_record(ctx, s))) return rc;
    if ((rc = download(ctx, dst, ctx->d_dst, out_bytes, s))) return rc;
    if (acc_debug && (rc = download(ctx, acc_debug, ctx->d_acc, out_bytes, s))) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return ENCHIP_OK;
}

int enchip_w8a8_batch(enchip_ctx *ctx, const float *a, int64_t M, int64_t K, const enchip_op *ops, int nops) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (nops < 0 || (nops > 0 && !ops)) return fail(ctx, ENCHIP_ERR_ARG, "batch: bad ops");
    if (M < 0 || M > ((int64_t)1 << 30) || K < 0) return fail(ctx, ENCHIP_ERR_ARG, "batch: bad shape");
    // Validate every op before any work (linalg/quant.go:330-339 does the same).
    std::vector<Weight *> ws((size_t)nops);
    for (int i = 0; i < nops; ++i) {
        int rc = find_weight(ctx, ops[i].w, &ws[(size_t)i]);
        if (rc) return rc;
        if (ws[(size_t)i]->K != K) return fail(ctx, ENCHIP_ERR_ARG, "batch: op %d has K=%lld, want %lld", i, (long long)ws[(size_t)i]->K, (long long)K);
        if (ops[i].act != ENCHIP_ACT_NONE && ops[i].act != ENCHIP_ACT_GELU) return fail(ctx, ENCHIP_ERR_ARG, "batch: bad act");
        if (!ops[i].dst) return fail(ctx, ENCHIP_ERR_ARG, "batch: op %d dst is NULL", i);
    }
    if (M == 0 || nops == 0) return ENCHIP_OK;
    if (K > 0 && !a) return fail(ctx, ENCHIP_ERR_ARG, "batch: a is NULL");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    const int64_t Kp = ws[0]->Kp;
    // each op has its own slice of the output and bias scratch, so every op is enqueued
    // before the one synchronisation at the end
    std::vector<int64_t> dst_off((size_t)nops), bias_off((size_t)nops);
    int64_t dst_total = 0, bias_total = 0;
    for (int i = 0; i < nops; ++i) {
        const int64_t n4 = round_up(ws[(size_t)i]->N, 4);  // 16-byte aligned slices
        dst_off[(size_t)i] = dst_total;
        bias_off[(size_t)i] = bias_total;
        dst_total += M * n4;
        bias_total += n4;
    }
    int rc;
    if ((rc = ensure(ctx, &ctx->d_a, &ctx->a_cap, (size_t)(M * K) * sizeof(float)))) return rc;
    if ((rc = ensure(ctx, &ctx->d_dst, &ctx->dst_cap, (size_t)dst_total * sizeof(float)))) return rc;
    if ((rc = ensure(ctx, &ctx->d_bias, &ctx->bias_cap, (size_t)bias_total * sizeof(float)))) return rc;
    if ((rc = ensure_act_scratch(ctx, M, Kp))) return rc;
    hipStream_t s = ctx->stream;
    if ((rc = scratch_wait(ctx, s))) return rc;
    if ((rc = upload(ctx, ctx->d_a, a, (size_t)(M * K) * sizeof(float), s))) return rc;
    // one quantization serves every op, so its layout must suit all of them
    bool af = true;
    for (int i = 0; i < nops; ++i)
        af = af && route_af(ctx, *ws[(size_t)i], M, ctx->d_dst + dst_off[(size_t)i], ws[(size_t)i]->N);
    if ((rc = launch_quant(ctx, ctx->d_a, M, K, ctx->d_aq, Kp, ctx->d_as, s, af))) return rc;
    for (int i = 0; i < nops; ++i) {
        const Weight &w = *ws[(size_t)i];
        float *db = ctx->d_bias + bias_off[(size_t)i], *dd = ctx->d_dst + dst_off[(size_t)i];
        if (ops[i].bias)
            HIP_TRY(ctx, hipMemcpyAsync(db, ops[i].bias, (size_t)w.N * sizeof(float), hipMemcpyHostToDevice, s));
        if ((rc = launch_gemm(ctx, w, ctx->d_aq, Kp, ctx->d_as, ops[i].bias ? db : nullptr, act_code(ops[i].act), dd,
                              w.N, M, s, af)))
            return rc;
    }
    if ((rc = scratch_record(ctx, s))) return rc;
    for (int i = 0; i < nops; ++i)
        if ((rc = download(ctx, ops[i].dst, ctx->d_dst + dst_off[(size_t)i],
                           (size_t)(M * ws[(size_t)i]->N) * sizeof(float), s)))
            return rc;
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return ENCHIP_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------- f32 MatmulBT

namespace {

// Enqueues C = A . B^T for count1 x count2 problems (gemm_f32.h), after the caller
// checked the arguments. Batches beyond the 65535 grid rows run as several launches.
int launch_matmul_f32(enchip_ctx *c, const float *A, int64_t lda, const float *B, int64_t ldb, bool bkn, float *C,
                      int64_t ldc, int64_t M, int64_t K, int64_t N, const enchip_f32_batch &b1,
                      const enchip_f32_batch &b2, hipStream_t s) {
    using namespace enchip;
    if (M == 0 || N == 0 || b1.count == 0 || b2.count == 0) return ENCHIP_OK;
    const F32Strides s1{b1.stride_a, b1.stride_b, b1.stride_c}, s2{b2.stride_a, b2.stride_b, b2.stride_c};
    auto al4 = [](int64_t v) { return v % 4 == 0; };
    const bool vec = K % 4 == 0 && al4(lda) && al4(s1.a) && al4(s2.a) && (uintptr_t)A % 16 == 0 &&
                     (bkn || (al4(ldb) && al4(s1.b) && al4(s2.b) && (uintptr_t)B % 16 == 0));
    const bool km = K % F32_KB != 0;
    // the LDS-staged kernel loads whole float4 of A rows and of B rows ([N,K]) or B k-rows ([K,N])
    const bool lds = K % 4 == 0 && al4(lda) && al4(s1.a) && al4(s2.a) && (uintptr_t)A % 16 == 0 && al4(ldb) &&
                     al4(s1.b) && al4(s2.b) && (uintptr_t)B % 16 == 0 && (!bkn || N % 4 == 0);
    const int wm = N <= 64 ? 4 : (M <= 64 ? 1 : 2), wn = 4 / wm;
    const int tilesM = (int)((M + 64 * wm - 1) / (64 * wm)), tilesN = (int)((N + 64 * wn - 1) / (64 * wn));
    constexpr int64_t kGrid = 65535;
    for (int64_t z0 = 0; z0 < b2.count; z0 += kGrid)
        for (int64_t y0 = 0; y0 < b1.count; y0 += kGrid) {
            const unsigned ny = (unsigned)std::min(kGrid, b1.count - y0), nz = (unsigned)std::min(kGrid, b2.count - z0);
            const float *a = A + y0 * s1.a + z0 * s2.a, *b = B + y0 * s1.b + z0 * s2.b;
            float *cz = C + y0 * s1.c + z0 * s2.c;
            if (K == 0) {  // whole rows per launch, at most 2^30 elements
                const int64_t rchunk = std::max<int64_t>(1, ((int64_t)1 << 30) / N);
                for (int64_t r0 = 0; r0 < M; r0 += rchunk) {
                    const int64_t n = std::min(rchunk, M - r0);
                    hipLaunchKernelGGL(fill_zero_f32, dim3((unsigned)((n * N + 255) / 256), ny, nz), dim3(256), 0, s,
                                       cz + r0 * ldc, ldc, s1.c, s2.c, (int)n, (int)N);
                }
                continue;
            }
            const dim3 grid((unsigned)(tilesM * tilesN), ny, nz), block(256);
            if (lds) {
                if (wm == 4 && bkn)
                    hipLaunchKernelGGL((gemm_f32_bt_lds<4, 1, true>), grid, block, 0, s, a, lda, b, ldb, cz, ldc, s1, s2,
                                       (int)M, (int)N, (int)K, tilesN);
                else if (wm == 4)
                    hipLaunchKernelGGL((gemm_f32_bt_lds<4, 1, false>), grid, block, 0, s, a, lda, b, ldb, cz, ldc, s1,
                                       s2, (int)M, (int)N, (int)K, tilesN);
                else if (wm == 1 && bkn)
                    hipLaunchKernelGGL((gemm_f32_bt_lds<1, 4, true>), grid, block, 0, s, a, lda, b, ldb, cz, ldc, s1, s2,
                                       (int)M, (int)N, (int)K, tilesN);
                else if (wm == 1)
                    hipLaunchKernelGGL((gemm_f32_bt_lds<1, 4, false>), grid, block, 0, s, a, lda, b, ldb, cz, ldc, s1,
                                       s2, (int)M, (int)N, (int)K, tilesN);
                else if (bkn)
                    hipLaunchKernelGGL((gemm_f32_bt_lds<2, 2, true>), grid, block, 0, s, a, lda, b, ldb, cz, ldc, s1, s2,
                                       (int)M, (int)N, (int)K, tilesN);
                else
                    hipLaunchKernelGGL((gemm_f32_bt_lds<2, 2, false>), grid, block, 0, s, a, lda, b, ldb, cz, ldc, s1,
                                       s2, (int)M, (int)N, (int)K, tilesN);
                continue;
            }
#define F32_CALL(WM, WN, BKN, VEC, KM)                                                                          \
    hipLaunchKernelGGL((gemm_f32_bt<WM, WN, BKN, VEC, KM>), grid, block, 0, s, a, lda, b, ldb, cz, ldc, s1, s2,   \
                       (int)M, (int)N, (int)K, tilesN)
#define F32_KM(WM, WN, BKN, VEC)                                                                               \
    do {                                                                                                       \
        if (km) F32_CALL(WM, WN, BKN, VEC, true);                                                              \
        else F32_CALL(WM, WN, BKN, VEC, false);                                                                \
    } while (0)
#define F32_LAUNCH(WM, WN)                                                                                     \
    do {                                                                                                       \
        if (bkn && vec) F32_KM(WM, WN, true, true);                                                            \
        else if (bkn) F32_KM(WM, WN, true, false);                                                             \
        else if (vec) F32_KM(WM, WN, false, true);                                                             \
        else F32_KM(WM, WN, false, false);                                                                     \
    } while (0)
            if (wm == 4) F32_LAUNCH(4, 1);
            else if (wm == 1) F32_LAUNCH(1, 4);
            else F32_LAUNCH(2, 2);
#undef F32_CALL
#undef F32_KM
#undef F32_LAUNCH
        }
    return check_launch(c, "gemm_f32_bt");
}

constexpr int64_t kMaxDimF32 = (int64_t)1 << 30;  // M, N, K; and M*N below 2^36 elements

}  // namespace

int enchip_matmul_bt_f32(enchip_ctx *ctx, const float *a, const float *b, float *dst, int64_t M, int64_t K, int64_t N) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (M < 0 || K < 0 || N < 0 || M > kMaxDimF32 || K > kMaxDimF32 || N > kMaxDimF32 || M * N > ((int64_t)1 << 36))
        return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_f32: bad shape M=%lld K=%lld N=%lld", (long long)M, (long long)K,
                    (long long)N);
    if (M == 0 || N == 0) return ENCHIP_OK;
    if (!dst || (K > 0 && (!a || !b))) return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_f32: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    int rc;
    const size_t out_bytes = (size_t)(M * N) * sizeof(float);
    if ((rc = ensure(ctx, &ctx->d_a, &ctx->a_cap, std::max<size_t>((size_t)(M * K) * sizeof(float), 16)))) return rc;
    if ((rc = ensure(ctx, &ctx->d_fb, &ctx->fb_cap, std::max<size_t>((size_t)(N * K) * sizeof(float), 16)))) return rc;
    if ((rc = ensure(ctx, &ctx->d_dst, &ctx->dst_cap, out_bytes))) return rc;
    hipStream_t s = ctx->stream;
    // operands are uploaded on every call: their contents are never cached (attention
    // rewrites pooled scratch in place between calls, gpu/enccuda/backend_test.go:88-130)
    if (K > 0) {
        if ((rc = upload(ctx, ctx->d_a, a, (size_t)(M * K) * sizeof(float), s))) return rc;
        if ((rc = upload(ctx, ctx->d_fb, b, (size_t)(N * K) * sizeof(float), s))) return rc;
    }
    const enchip_f32_batch one{1, 0, 0, 0};
    if ((rc = launch_matmul_f32(ctx, ctx->d_a, K, ctx->d_fb, K, false, ctx->d_dst, N, M, K, N, one, one, s))) return rc;
    if ((rc = download(ctx, dst, ctx->d_dst, out_bytes, s))) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return ENCHIP_OK;
}

int enchip_matmul_bt_f32_dev(enchip_ctx *ctx, const float *d_a, int64_t lda, const float *d_b, int64_t ldb,
                             int b_layout, float *d_c, int64_t ldc, int64_t M, int64_t K, int64_t N,
                             const enchip_f32_batch *inner, const enchip_f32_batch *outer, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (b_layout != ENCHIP_B_NK && b_layout != ENCHIP_B_KN)
        return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_f32_dev: bad b_layout %d", b_layout);
    const bool bkn = b_layout == ENCHIP_B_KN;
    const enchip_f32_batch one{1, 0, 0, 0};
    const enchip_f32_batch b1 = inner ? *inner : one, b2 = outer ? *outer : one;
    if (M < 0 || K < 0 || N < 0 || M > kMaxDimF32 || K > kMaxDimF32 || N > kMaxDimF32 ||
        M * N > ((int64_t)1 << 36) || b1.count < 0 || b2.count < 0 || b1.count > kMaxDimF32 || b2.count > kMaxDimF32)
        return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_f32_dev: bad shape M=%lld K=%lld N=%lld batch %lld x %lld",
                    (long long)M, (long long)K, (long long)N, (long long)b1.count, (long long)b2.count);
    if (M == 0 || N == 0 || b1.count == 0 || b2.count == 0) return ENCHIP_OK;
    if (lda < K || ldb < (bkn ? N : K) || ldc < N)
        return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_f32_dev: pitches lda=%lld ldb=%lld ldc=%lld must cover a row (K=%lld, N=%lld)",
                    (long long)lda, (long long)ldb, (long long)ldc, (long long)K, (long long)N);
    for (const enchip_f32_batch *b : {&b1, &b2})
        if (b->stride_a < 0 || b->stride_b < 0 || b->stride_c < 0)
            return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_f32_dev: batch strides must be >= 0");
    if (!d_c || (K > 0 && (!d_a || !d_b))) return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_f32_dev: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    return launch_matmul_f32(ctx, d_a, lda, d_b, ldb, bkn, d_c, ldc, M, K, N, b1, b2, s);
}

// ---------------------------------------------------------------------------- weight-only int8 MatmulBTQ8

namespace {

// Enqueues C = A . (f32(q) * wscale)^T for a registered weight (gemm_q8w.h), after the
// caller checked the arguments. K = 0 gives zeros (an empty sum, whatever the scales).
int launch_matmul_q8w(enchip_ctx *c, const Weight &w, const float *A, int64_t lda, float *C, int64_t ldc,
                      int64_t M, hipStream_t s) {
    using namespace enchip;
    if (M == 0) return ENCHIP_OK;
    if (w.K == 0) {
        const int64_t rchunk = std::max<int64_t>(1, ((int64_t)1 << 30) / w.N);
        for (int64_t r0 = 0; r0 < M; r0 += rchunk) {
            const int64_t n = std::min(rchunk, M - r0);
            hipLaunchKernelGGL(fill_zero_f32, dim3((unsigned)((n * w.N + 255) / 256)), dim3(256), 0, s, C + r0 * ldc,
                               ldc, (int64_t)0, (int64_t)0, (int)n, (int)w.N);
        }
        return check_launch(c, "fill_zero_f32");
    }
    const bool vec = w.K % 4 == 0 && lda % 4 == 0 && (uintptr_t)A % 16 == 0;
    // 128 x 256 tiles when they give every CU two workgroups, else 128 x 128 when those
    // do, else 64 x 64 when those give every CU one; below that the K-split small form
    // (32 x 64 tiles, or 32 x 32 when 32 x 64 would leave CUs idle). Measured on MI355X:
    // M = 512, K = 768, N = 2304 takes 24 us as 288 64 x 64 tiles against 31 in the small
    // form, which re-splits A for each column tile; M = 128, K = 768, N = 768, 24 such
    // tiles, takes 18 us against 9.
    const int64_t cus = c->num_cus, cus2 = 2 * cus;
    auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((w.N + bn - 1) / bn); };
    const int form = tiles(128, 256) >= cus2 ? 2 : tiles(128, 128) >= cus2 ? 1 : tiles(64, 64) >= cus ? 0
                     : tiles(32, 64) >= cus ? -2 : -1;
    const bool wide = form > 0;
    const int bm = form < 0 ? 32 : wide ? 128 : 64, bn = form == 2 ? 256 : form == -2 ? 64 : form == -1 ? 32 : bm;
    const int tilesN = (int)((w.N + bn - 1) / bn);
    // every wavefront reads whole 32-channel blocks of the image up to tilesN * bn
    if ((int64_t)tilesN * bn > w.Np) return fail(c, ENCHIP_ERR_ARG, "gemm_q8w: %d tiles exceed the image", tilesN);
    // rows per launch: at most 2^30 / tilesN tiles of rows, so the tile index stays an int
    const int64_t rows = std::max<int64_t>(bm, (((int64_t)1 << 30) / tilesN) / bm * bm);
    for (int64_t r0 = 0; r0 < M; r0 += rows) {
        const int64_t n = std::min(rows, M - r0);
        const dim3 grid((unsigned)(((n + bm - 1) / bm) * tilesN)), block(256);
        const float *a = A + r0 * lda;
        float *cz = C + r0 * ldc;
#define Q8W_CALL(TM, TN, VEC)                                                                                   \
    hipLaunchKernelGGL((gemm_q8w<TM, TN, VEC>), grid, block, 0, s, a, lda, w.d_w, w.d_s, cz, ldc, (int)n,       \
                       (int)w.N, (int)w.K, (int)w.Kp, tilesN)
#define Q8W_SMALL(TN, VEC)                                                                                      \
    hipLaunchKernelGGL((gemm_q8w_small<TN, VEC>), grid, block, 0, s, a, lda, w.d_w, w.d_s, cz, ldc, (int)n,     \
                       (int)w.N, (int)w.K, (int)w.Kp, tilesN)
        if (form == -2 && vec) Q8W_SMALL(2, true);
        else if (form == -2) Q8W_SMALL(2, false);
        else if (form == -1 && vec) Q8W_SMALL(1, true);
        else if (form == -1) Q8W_SMALL(1, false);
        else if (form == 2 && vec) Q8W_CALL(2, 4, true);
        else if (form == 2) Q8W_CALL(2, 4, false);
        else if (wide && vec) Q8W_CALL(2, 2, true);
        else if (wide) Q8W_CALL(2, 2, false);
        else if (vec) Q8W_CALL(1, 1, true);
        else Q8W_CALL(1, 1, false);
#undef Q8W_CALL
#undef Q8W_SMALL
    }
    return check_launch(c, "gemm_q8w");
}

// The shared argument checks of the two entry points.
int check_q8w(enchip_ctx *c, const char *what, const Weight &w, int64_t M) {
    if (M < 0 || M > kMaxDimF32 || M * w.N > ((int64_t)1 << 36))
        return fail(c, ENCHIP_ERR_ARG, "%s: bad M=%lld for N=%lld", what, (long long)M, (long long)w.N);
    // The sum is scaled once at the end (inf * sum), where the CPU path scales each weight
    // first (f32(q) * inf, NaN for a zero code): the two differ, so such a weight declines.
    if (w.inf_scale)
        return fail(c, ENCHIP_ERR_ARG, "%s: the weight has an infinite scale (the CPU path handles it)", what);
    return ENCHIP_OK;
}

}  // namespace

int enchip_matmul_bt_q8(enchip_ctx *ctx, enchip_weight h, const float *a, int64_t M, float *dst) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if ((rc = check_q8w(ctx, "matmul_bt_q8", *w, M))) return rc;
    if (M == 0) return ENCHIP_OK;
    if (!dst || (w->K > 0 && !a)) return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_q8: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    const size_t in_bytes = (size_t)(M * w->K) * sizeof(float), out_bytes = (size_t)(M * w->N) * sizeof(float);
    if ((rc = ensure(ctx, &ctx->d_a, &ctx->a_cap, std::max<size_t>(in_bytes, 16)))) return rc;
    if ((rc = ensure(ctx, &ctx->d_dst, &ctx->dst_cap, out_bytes))) return rc;
    hipStream_t s = ctx->stream;
    // the activations are uploaded on every call (gpu/enccuda/backend.go:271-275)
    if ((rc = upload(ctx, ctx->d_a, a, in_bytes, s))) return rc;
    if ((rc = launch_matmul_q8w(ctx, *w, ctx->d_a, w->K, ctx->d_dst, w->N, M, s))) return rc;
    if ((rc = download(ctx, dst, ctx->d_dst, out_bytes, s))) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return ENCHIP_OK;
}

int enchip_matmul_bt_q8_dev(enchip_ctx *ctx, enchip_weight h, const float *d_a, int64_t lda, int64_t M,
                            float *d_dst, int64_t ldd, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if ((rc = check_q8w(ctx, "matmul_bt_q8_dev", *w, M))) return rc;
    if (M == 0) return ENCHIP_OK;
    if (lda < w->K || ldd < w->N)
        return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_q8_dev: pitches lda=%lld ldd=%lld must cover a row (K=%lld, N=%lld)",
                    (long long)lda, (long long)ldd, (long long)w->K, (long long)w->N);
    if (!d_dst || (w->K > 0 && !d_a)) return fail(ctx, ENCHIP_ERR_ARG, "matmul_bt_q8_dev: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    return launch_matmul_q8w(ctx, *w, d_a, lda, d_dst, ldd, M, s);
}

// ---------------------------------------------------------------------------- encoder row ops

namespace {

constexpr int64_t kMaxRowOp = 4096;  // softmax columns / LayerNorm width held in registers

// Launches K<CPL> for rows of up to 64*CPL floats, CPL the smallest power of two that fits.
#define ROWOP_DISPATCH(KERNEL, n, grid, s, ...)                                               \
    do {                                                                                     \
        if ((n) <= 64) hipLaunchKernelGGL((KERNEL<1>), grid, dim3(256), 0, s, __VA_ARGS__);    \
        else if ((n) <= 128) hipLaunchKernelGGL((KERNEL<2>), grid, dim3(256), 0, s, __VA_ARGS__); \
        else if ((n) <= 256) hipLaunchKernelGGL((KERNEL<4>), grid, dim3(256), 0, s, __VA_ARGS__); \
        else if ((n) <= 512) hipLaunchKernelGGL((KERNEL<8>), grid, dim3(256), 0, s, __VA_ARGS__); \
        else if ((n) <= 1024) hipLaunchKernelGGL((KERNEL<16>), grid, dim3(256), 0, s, __VA_ARGS__); \
        else if ((n) <= 2048) hipLaunchKernelGGL((KERNEL<32>), grid, dim3(256), 0, s, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<64>), grid, dim3(256), 0, s, __VA_ARGS__);            \
    } while (0)

}  // namespace

int enchip_softmax_rows_scaled_dev(enchip_ctx *ctx, float *d_x, int64_t ld, int64_t rows, int64_t cols, float scale,
                                   void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (rows < 0 || cols < 0 || cols > kMaxRowOp || ld < cols)
        return fail(ctx, ENCHIP_ERR_ARG, "softmax: bad shape rows=%lld cols=%lld ld=%lld (cols <= %lld)",
                    (long long)rows, (long long)cols, (long long)ld, (long long)kMaxRowOp);
    if (rows == 0 || cols == 0) return ENCHIP_OK;
    if (!d_x) return fail(ctx, ENCHIP_ERR_ARG, "softmax: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    for (int64_t r0 = 0; r0 < rows; r0 += kRowChunk) {
        const int64_t n = std::min(kRowChunk, rows - r0);
        const dim3 grid((unsigned)((n + 3) / 4));
        ROWOP_DISPATCH(enchip::softmax_rows_scaled, cols, grid, s, d_x + r0 * ld, ld, n, (int)cols, scale);
    }
    return check_launch(ctx, "softmax_rows_scaled");
}

int enchip_residual_layer_norm_dev(enchip_ctx *ctx, float *d_h, int64_t ldh, const float *d_y, int64_t ldy,
                                   int64_t rows, int64_t D, const float *d_w, const float *d_b, double eps,
                                   void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (rows < 0 || D < 0 || D > kMaxRowOp || ldh < D || (d_y && ldy < D))
        return fail(ctx, ENCHIP_ERR_ARG, "layer_norm: bad shape rows=%lld D=%lld ldh=%lld ldy=%lld (D <= %lld)",
                    (long long)rows, (long long)D, (long long)ldh, (long long)ldy, (long long)kMaxRowOp);
    if (rows == 0 || D == 0) return ENCHIP_OK;
    if (!d_h || !d_w || !d_b) return fail(ctx, ENCHIP_ERR_ARG, "layer_norm: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    const bool vec = D % 4 == 0 && ldh % 4 == 0 && (!d_y || ldy % 4 == 0) && (uintptr_t)d_h % 16 == 0 &&
                     (uintptr_t)d_y % 16 == 0 && (uintptr_t)d_w % 16 == 0 && (uintptr_t)d_b % 16 == 0 && D >= 4;
    for (int64_t r0 = 0; r0 < rows; r0 += kRowChunk) {
        const int64_t n = std::min(kRowChunk, rows - r0);
        const dim3 grid((unsigned)((n + 3) / 4));
        float *h = d_h + r0 * ldh;
        const float *y = d_y ? d_y + r0 * ldy : nullptr;
    // VEC: 4 consecutive columns per lane per 16-byte load (CPL a multiple of 4)
#define LN_CASE(CPL)                                                                                           \
    do {                                                                                                       \
        if (vec)                                                                                               \
            hipLaunchKernelGGL((enchip::residual_layer_norm<CPL, true>), grid, dim3(256), 0, s, h, ldh, y, ldy, n, \
                               (int)D, d_w, d_b, eps);                                                          \
        else                                                                                                   \
            hipLaunchKernelGGL((enchip::residual_layer_norm<CPL, false>), grid, dim3(256), 0, s, h, ldh, y, ldy, n, \
                               (int)D, d_w, d_b, eps);                                                          \
    } while (0)
        if (D <= 64 && !vec) LN_CASE(1);
        else if (D <= 128 && !vec) LN_CASE(2);
        else if (D <= 256) LN_CASE(4);
        else if (D <= 512) LN_CASE(8);
        else if (D <= 768) LN_CASE(12);  // BERT-base: 3 float4 per lane, none idle
        else if (D <= 1024) LN_CASE(16);
        else if (D <= 2048) LN_CASE(32);
        else LN_CASE(64);
#undef LN_CASE
    }
    return check_launch(ctx, "residual_layer_norm");
}

int enchip_residual_layer_norm_quant_dev(enchip_ctx *ctx, float *d_h, int64_t ldh, const float *d_y, int64_t ldy,
                                         int64_t rows, int64_t D, const float *d_w, const float *d_b, double eps,
                                         int8_t *d_aq, int64_t ldq, float *d_ascale, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (rows < 0 || D < 4 || D > kMaxRowOp || D % 4 != 0 || ldh < D || ldh % 4 != 0 || (d_y && (ldy < D || ldy % 4 != 0)) ||
        ldq < D || ldq % 64 != 0 || ldq > kMaxRowOp)
        return fail(ctx, ENCHIP_ERR_ARG,
                    "layer_norm_quant: bad shape rows=%lld D=%lld ldh=%lld ldy=%lld ldq=%lld (D a multiple of 4, "
                    "pitches multiples of 4, ldq a multiple of 64 in [D, %lld])",
                    (long long)rows, (long long)D, (long long)ldh, (long long)ldy, (long long)ldq, (long long)kMaxRowOp);
    if (rows == 0) return ENCHIP_OK;
    if (!d_h || !d_w || !d_b || !d_aq || !d_ascale) return fail(ctx, ENCHIP_ERR_ARG, "layer_norm_quant: null pointer");
    if ((uintptr_t)d_h % 16 || (uintptr_t)d_y % 16 || (uintptr_t)d_w % 16 || (uintptr_t)d_b % 16 || (uintptr_t)d_aq % 16)
        return fail(ctx, ENCHIP_ERR_ARG, "layer_norm_quant: h, y, w, b and aq must be 16-byte aligned");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    const int64_t width = std::max(D, ldq);
    // chunks of kRowChunk rows (a multiple of 32: fragment-major rows r0.. start at r0 * ldq)
    for (int64_t r0 = 0; r0 < rows; r0 += kRowChunk) {
        const int64_t n = std::min(kRowChunk, rows - r0);
        const dim3 grid((unsigned)((n + 7) / 8));
        float *h = d_h + r0 * ldh;
        const float *y = d_y ? d_y + r0 * ldy : nullptr;
        int8_t *aq = d_aq + r0 * ldq;
        float *as = d_ascale + r0;
#define LNQ_CASE(CPL)                                                                                          \
    hipLaunchKernelGGL((enchip::residual_layer_norm_quant<CPL>), grid, dim3(512), 0, s, h, ldh, y, ldy, n, (int)D, \
                       d_w, d_b, eps, aq, ldq, as)
        if (width <= 256) LNQ_CASE(4);
        else if (width <= 512) LNQ_CASE(8);
        else if (width <= 768) LNQ_CASE(12);  // BERT-base: 3 float4 per lane, none idle
        else if (width <= 1024) LNQ_CASE(16);
        else if (width <= 2048) LNQ_CASE(32);
        else LNQ_CASE(64);
#undef LNQ_CASE
    }
    return check_launch(ctx, "residual_layer_norm_quant");
}

int enchip_pool_mean_l2_dev(enchip_ctx *ctx, const float *d_h, int64_t ldh, int64_t nseq, int64_t L, int64_t D,
                            float *d_out, int64_t ldo, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (nseq < 0 || L < 0 || D < 0 || D > 4096 || ldh < D || ldo < D || nseq > 65535 || L > 0x7fffffff)
        return fail(ctx, ENCHIP_ERR_ARG, "pool: bad shape nseq=%lld L=%lld D=%lld (D <= 4096, nseq <= 65535)",
                    (long long)nseq, (long long)L, (long long)D);
    if (nseq == 0 || D == 0) return ENCHIP_OK;
    if (!d_out || (L > 0 && !d_h)) return fail(ctx, ENCHIP_ERR_ARG, "pool: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    hipLaunchKernelGGL(enchip::pool_mean_cols, dim3((unsigned)((D + 255) / 256), (unsigned)nseq), dim3(256), 0, s, d_h,
                       ldh, (int)L, (int)D, d_out, ldo);
    hipLaunchKernelGGL(enchip::l2_normalize_rows, dim3((unsigned)nseq), dim3(256), 0, s, d_out, ldo, (int)D);
    return check_launch(ctx, "pool_mean_l2");
}

int enchip_attention_f32_dev(enchip_ctx *ctx, const float *d_q, const float *d_k, const float *d_v, int64_t ld,
                             float *d_out, int64_t ldo, int64_t nseq, int64_t L, int64_t heads, int64_t head_dim,
                             float scale, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    const bool flash = ctx->att_products == ENCHIP_ATT_FLASH_BF16 || ctx->att_products == ENCHIP_ATT_FLASH_F16;
    const bool f16 = ctx->att_products == ENCHIP_ATT_FLASH_F16;
    if (head_dim != 32 && head_dim != 64)
        return fail(ctx, ENCHIP_ERR_ARG, "attention: head_dim must be 32 or 64, got %lld", (long long)head_dim);
    const int64_t max_l = flash ? ((int64_t)1 << 30) : enchip::ATT_MAX_L;
    if (nseq < 0 || L < 0 || L > max_l || heads < 0 || heads > 65535 || ld < heads * head_dim ||
        ldo < heads * head_dim || ld % 4 != 0 || nseq * L > ((int64_t)1 << 31) ||
        (flash && ld > INT32_MAX / enchip::FA_KT))  // the flash kernel's 32-bit in-tile offsets
        return fail(ctx, ENCHIP_ERR_ARG,
                    "attention: bad shape nseq=%lld L=%lld (<= %lld in this product mode) heads=%lld ld=%lld ldo=%lld "
                    "(ld a multiple of 4 covering heads*head_dim, below 2^25 in the flash mode)",
                    (long long)nseq, (long long)L, (long long)max_l, (long long)heads, (long long)ld, (long long)ldo);
    if (nseq == 0 || L == 0 || heads == 0) return ENCHIP_OK;
    if (!d_q || !d_k || !d_v || !d_out) return fail(ctx, ENCHIP_ERR_ARG, "attention: null pointer");
    if ((uintptr_t)d_q % 16 || (uintptr_t)d_k % 16 || (uintptr_t)d_v % 16)
        return fail(ctx, ENCHIP_ERR_ARG, "attention: q, k and v must be 16-byte aligned");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    using Kern = void (*)(const float *, const float *, const float *, int64_t, float *, int64_t, int, int, float);
    Kern fn;
    size_t lds;
    int64_t per_seq, threads;
    if (flash) {
        const bool vec = ldo % 4 == 0 && (uintptr_t)d_out % 16 == 0;
        constexpr int nw8 = enchip::FA_WAVES, nw16 = enchip::FA_WAVES_WIDE;
        // 16 wavefronts once L > 256, except:
        //  - L = 512 (two full 8-wavefront workgroups per head): two workgroups per CU
        //    whose barrier phases drift apart overlap one's MFMA work with the other's
        //    softmax, which outweighs splitting each K / V tile twice (BERT-base, 64 x 12
        //    heads: 190-194 -> 175-177 us; XLM-R-large, 128 x 16: 490 -> 472-477);
        //  - L > 512 on a grid with fewer workgroups than CUs: the 8-wavefront form's
        //    twice as many workgroups spread further (L = 1000 over 8 heads x sequences:
        //    51 against 78 us).
        // Otherwise up to L = 512 one 16-wavefront workgroup covers a head's queries that
        // two 8-wavefront ones would split unevenly (L = 300 over 768 heads x sequences:
        // 94.5 against 98.7 us). The results are the same bits either way.
        const int64_t wide_grid = ((L + 32 * nw16 - 1) / (32 * nw16)) * heads * nseq;
        const bool wide = L > enchip::FA_WIDE_L &&
                          (L <= 32 * nw16 ? L != 32 * nw16 : wide_grid >= ctx->num_cus);
        const int nw = wide ? nw16 : nw8;
        lds = (size_t)enchip::fa_lds_bytes((int)head_dim);
        per_seq = ((L + 32 * nw - 1) / (32 * nw)) * heads;
        threads = 64 * nw;
#define FA_PICK(F16)                                                                                          \
    (wide ? (head_dim == 64 ? (vec ? enchip::attention_flash<64, nw16, true, F16> : enchip::attention_flash<64, nw16, false, F16>) \
                            : (vec ? enchip::attention_flash<32, nw16, true, F16> : enchip::attention_flash<32, nw16, false, F16>)) \
          : (head_dim == 64 ? (vec ? enchip::attention_flash<64, nw8, true, F16> : enchip::attention_flash<64, nw8, false, F16>) \
                            : (vec ? enchip::attention_flash<32, nw8, true, F16> : enchip::attention_flash<32, nw8, false, F16>)))
        fn = f16 ? FA_PICK(true) : FA_PICK(false);
#undef FA_PICK
    } else {
        const bool split = ctx->att_products == ENCHIP_ATT_SPLIT_BF16;
        const bool full = L == enchip::ATT_MAX_L;
        lds = (size_t)(split ? enchip::att_split_lds_floats((int)L) : enchip::att_lds_floats((int)L)) * sizeof(float);
        per_seq = ((L + enchip::ATT_QT - 1) / enchip::ATT_QT) * heads;
        threads = 64 * enchip::ATT_WAVES;
        fn = split ? (head_dim == 64 ? (full ? enchip::attention_split_bf16<64, true>
                                             : enchip::attention_split_bf16<64, false>)
                                     : (full ? enchip::attention_split_bf16<32, true>
                                             : enchip::attention_split_bf16<32, false>))
                   : (head_dim == 64 ? enchip::attention_f32<64> : enchip::attention_f32<32>);
    }
    const std::pair<const void *, size_t> key(reinterpret_cast<const void *>(fn), lds);
    if (std::find(ctx->lds_set.begin(), ctx->lds_set.end(), key) == ctx->lds_set.end()) {
        HIP_TRY(ctx, hipFuncSetAttribute(key.first, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        ctx->lds_set.push_back(key);
    }
    // one launch per chunk of sequences whose global thread index fits 32 bits
    const int64_t chunk = std::max<int64_t>(1, ((((int64_t)1 << 32) - 1) / threads) / per_seq);
    for (int64_t z0 = 0; z0 < nseq; z0 += chunk) {
        const int64_t nz = std::min<int64_t>(chunk, nseq - z0);
        const dim3 grid((unsigned)(per_seq * nz));
        const int64_t off = z0 * L;
        hipLaunchKernelGGL(fn, grid, dim3((unsigned)threads), lds, s, d_q + off * ld, d_k + off * ld, d_v + off * ld,
                           ld, d_out + off * ldo, ldo, (int)L, (int)heads, scale);
    }
    return check_launch(ctx, flash ? "attention_flash" : "attention");
}

int enchip_set_attention_products(enchip_ctx *ctx, int mode) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (mode != ENCHIP_ATT_F32 && mode != ENCHIP_ATT_SPLIT_BF16 && mode != ENCHIP_ATT_FLASH_BF16 &&
        mode != ENCHIP_ATT_FLASH_F16)
        return fail(ctx, ENCHIP_ERR_ARG, "attention products: mode must be ENCHIP_ATT_F32, ENCHIP_ATT_SPLIT_BF16, "
                    "ENCHIP_ATT_FLASH_BF16 or ENCHIP_ATT_FLASH_F16");
    ctx->att_products = mode;
    return ENCHIP_OK;
}

// ---------------------------------------------------------------------------- top-k

namespace {

// Stage-1 chunks (rows x chunks) from which the threshold filter runs: below it the
// threshold's two extra dependent launches cost more than the selections they skip.
// Measured on MI355X at n = 2^20 (128 chunks per row), k = 10, per call: 32 rows 57 ->
// 63 us with the filter, 64 rows 91 -> 81, 256 rows 291 -> 207.
constexpr int64_t kTopkFilterChunks = 8192;
// The same floor for the radix stage 1 (k > 64, 4096-score chunks), whose selections cost
// more: at n = 2^20 (256 chunks per row), k = 100, per call, 16 rows 151 -> 127 us with the
// filter, 8 rows 126 -> 120, 4 rows 117 either way; 256 rows 847 -> 375.
constexpr int64_t kTopkFilterChunksRadix = 1024;

// The per-row bounds from the first TOPK_SAMPLE_CHUNKS chunks' candidates (cr, nr rows of
// nchunks * k): topk_thresh's wavefront rounds up to k = TOPK_SORT_K, a sort above.
void launch_thresh(const uint64_t *cr, int64_t nr, int64_t nchunks, int64_t k, uint64_t *thr, unsigned *zero,
                   hipStream_t s) {
    using namespace enchip;
    if (k > TOPK_SORT_K)
        hipLaunchKernelGGL(topk_thresh_sorted, dim3((unsigned)nr), dim3(256), 0, s, cr, (int)nchunks, (int)k, thr,
                           zero);
    else
        hipLaunchKernelGGL(topk_thresh, dim3((unsigned)((nr + 3) / 4)), dim3(256), 0, s, cr, nr, (int)nchunks, (int)k,
                           thr, zero);
}

// Enqueues the two top-k stages (topk.h) after the caller checked the arguments.
int launch_topk(enchip_ctx *c, const float *scores, int64_t ld, int64_t rows, int64_t n, int64_t k, int32_t *index,
                int64_t ldi, float *score, int64_t lds, hipStream_t s) {
    using namespace enchip;
    if (rows == 0 || k == 0) return ENCHIP_OK;
    if (n == 0) {  // no candidates: the merge pads every row (-1, NaN)
        hipLaunchKernelGGL(topk_empty, dim3((unsigned)std::min<int64_t>(rows, 65535)), dim3(256), 0, s, rows, (int)k,
                           index, ldi, score, lds);
        return check_launch(c, "topk");
    }
    // Long rows on a grid of many chunks: threshold from each row's first chunks, then the
    // other chunks filter against it (topk_chunk_wide), so most skip their selection. The
    // thresholds (one key per row) follow the candidates in the scratch.
    // topk_chunk_wide up to k = 64, else the radix topk_chunk. Measured on MI355X at n = 2^20
    // (same process, per call), against the radix stage 1: k = 64 at 1, 16, 256 rows 81, 119,
    // 765 -> 40, 70, 238 us; k = 33 61, 98, 756 -> 36, 63, 226 us.
    const bool wide = k <= TOPK_WIDE_K;
    const int64_t chunk = wide ? TOPK_WCHUNK : TOPK_CHUNK;
    const int64_t nchunks = std::max<int64_t>(1, (n + chunk - 1) / chunk);
    const bool filter =
        nchunks >= 2 * TOPK_SAMPLE_CHUNKS && rows * nchunks >= (wide ? kTopkFilterChunks : kTopkFilterChunksRadix);
    int rc;
    if ((rc = ensure(c, &c->d_cand, &c->cand_cap, (size_t)(rows * nchunks * k + (filter ? rows : 0)) * sizeof(uint64_t))))
        return rc;
    uint64_t *thr = filter ? c->d_cand + rows * nchunks * k : nullptr;
    int kp = 1;
    while (kp < k) kp <<= 1;
    for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
        const int64_t nr = std::min<int64_t>(65535, rows - r0);
        uint64_t *cr = c->d_cand + r0 * nchunks * k;
        if (filter && wide) {
            hipLaunchKernelGGL(topk_chunk_wide, dim3((unsigned)TOPK_SAMPLE_CHUNKS, (unsigned)nr), dim3(256), 0, s,
                               scores + r0 * ld, ld, n, (int)k, (int)nchunks, cr, 0, (const uint64_t *)nullptr);
            launch_thresh(cr, nr, nchunks, k, thr + r0, nullptr, s);
            hipLaunchKernelGGL(topk_chunk_wide, dim3((unsigned)(nchunks - TOPK_SAMPLE_CHUNKS), (unsigned)nr), dim3(256), 0,
                               s, scores + r0 * ld, ld, n, (int)k, (int)nchunks, cr, TOPK_SAMPLE_CHUNKS,
                               (const uint64_t *)(thr + r0));
        } else if (wide) {
            hipLaunchKernelGGL(topk_chunk_wide, dim3((unsigned)nchunks, (unsigned)nr), dim3(256), 0, s, scores + r0 * ld,
                               ld, n, (int)k, (int)nchunks, cr, 0, (const uint64_t *)nullptr);
        } else if (filter) {
            hipLaunchKernelGGL(topk_chunk, dim3((unsigned)TOPK_SAMPLE_CHUNKS, (unsigned)nr), dim3(256), 0, s,
                               scores + r0 * ld, ld, n, (int)k, (int)nchunks, cr, 0, (const uint64_t *)nullptr);
            hipLaunchKernelGGL(topk_thresh_radix, dim3((unsigned)nr), dim3(256), 0, s, (const uint64_t *)cr,
                               (int)nchunks, (int)k, thr + r0);
            hipLaunchKernelGGL(topk_chunk, dim3((unsigned)(nchunks - TOPK_SAMPLE_CHUNKS), (unsigned)nr), dim3(256), 0, s,
                               scores + r0 * ld, ld, n, (int)k, (int)nchunks, cr, TOPK_SAMPLE_CHUNKS,
                               (const uint64_t *)(thr + r0));
        } else {
            hipLaunchKernelGGL(topk_chunk, dim3((unsigned)nchunks, (unsigned)nr), dim3(256), 0, s, scores + r0 * ld, ld,
                               n, (int)k, (int)nchunks, cr, 0, (const uint64_t *)nullptr);
        }
    }
    for (int64_t r0 = 0; r0 < rows; r0 += kRowChunk) {
        const int64_t nr = std::min<int64_t>(kRowChunk, rows - r0);
        hipLaunchKernelGGL(topk_merge, dim3((unsigned)nr), dim3(256), (size_t)kp * sizeof(uint64_t), s,
                           c->d_cand + r0 * nchunks * k, nchunks * k, (int)k, kp, scores + r0 * ld, ld,
                           index + r0 * ldi, ldi, score + r0 * lds, lds);
    }
    return check_launch(c, "topk");
}

// enchip_ann_topk's fused route: the selection runs in the scoring GEMM's epilogue, so the
// M x N scores are never written or read back.
//   1. gemm_w8a8_pt scores each row's first kSinkSample columns into d_dst, and stage 1
//      + topk_thresh take the k-th largest key among them: a lower bound of the row's
//      k-th largest key (the sample is part of the row). topk_thresh zeroes the counts.
//   2. gemm_w8a8_pt<EPI_TOPK> scores every column and appends the scores whose key is at
//      or above their row's bound to the row's list (gemm_persistent.h, TopkSink): the
//      row's k largest keys are all there.
//   3. topk_sink_merge selects the k largest of each list.
// About k of every kSinkSample columns clear a bound on exchangeable scores (k * N /
// kSinkSample per row); a row whose list overflows its capacity (sink_cap: adversarial
// orders, e.g. scores rising along the index) makes the caller run the two-pass route
// instead.
constexpr int64_t kSinkSample = (int64_t)enchip::TOPK_SAMPLE_CHUNKS * enchip::TOPK_WCHUNK;

// Candidates listed per row: 4096 for k <= 32, 8192 for k <= 64 (topk_sink_merge holds
// them 16 or 32 per thread).
int sink_cap(int64_t k) { return k <= enchip::TOPK_SMALL_K ? enchip::TOPK_CHUNK : 2 * enchip::TOPK_CHUNK; }

// k <= TOPK_WIDE_K over rows at least 4 samples long whose expected lists fill at most a
// quarter of the capacity, on fragment-major activations: the linear route's own (af), or, for
// M at or below the small-M limit, quantized fragment-major for this route alone when the
// skinny candidate kernel and the persistent GEMM (sample scores, two-pass fallback) take
// the shape.
bool ann_fused_ok(const enchip_ctx *c, const Weight &w, int64_t M, int64_t k, bool af) {
    if (k < 1 || k > enchip::TOPK_WIDE_K || w.N < 4 * kSinkSample || k * w.N > (int64_t)sink_cap(k) * kSinkSample / 4)
        return false;
    // from 8 queries: measured on MI355X (2^20 x 384, k = 10, per host call) M = 16 207 -> 189 us,
    // M = 1 150 -> 179 us (the GEMV's scores are cheap there, the extra launches are not)
    return af || (M >= 8 && M <= c->small_m && skinny_shape_nk(w, nullptr, w.Kp, true) != 0 &&
                  use_persistent(w, nullptr, w.Kp, nullptr, w.N, M, true));
}

// Enqueues steps 1-3 on s for M rows of fragment-major codes in the context scratch
// (d_aq, d_as), leaving the hits at hit_i / hit_s (M x k each) and the list sizes at
// count (M), all device memory.
int launch_ann_fused(enchip_ctx *c, const Weight &w, int64_t M, int64_t k, hipStream_t s, int32_t *hit_i,
                     float *hit_s, unsigned *count) {
    using namespace enchip;
    int rc;
    if ((rc = ensure(c, &c->d_dst, &c->dst_cap, (size_t)(M * kSinkSample) * sizeof(float)))) return rc;
    const int64_t cand_n = M * TOPK_SAMPLE_CHUNKS * k, cap = sink_cap(k);
    const size_t words = (size_t)(cand_n + M + M * cap) + (size_t)(M * cap + 1) / 2;
    if ((rc = ensure(c, &c->d_cand, &c->cand_cap, words * sizeof(uint64_t)))) return rc;
    uint64_t *cand = c->d_cand, *thr = cand + cand_n, *keys = thr + M;
    float *raw = reinterpret_cast<float *>(keys + M * cap);
    Weight sample = w;
    sample.N = sample.Np = kSinkSample;
    if ((rc = launch_gemm(c, sample, c->d_aq, w.Kp, c->d_as, nullptr, EPI_F32, c->d_dst, kSinkSample, M, s, true)))
        return rc;
    for (int64_t r0 = 0; r0 < M; r0 += 65535) {
        const int64_t nr = std::min<int64_t>(65535, M - r0);
        uint64_t *cr = cand + r0 * TOPK_SAMPLE_CHUNKS * k;
        hipLaunchKernelGGL(topk_chunk_wide, dim3((unsigned)TOPK_SAMPLE_CHUNKS, (unsigned)nr), dim3(256), 0, s,
                           c->d_dst + r0 * kSinkSample, kSinkSample, kSinkSample, (int)k, TOPK_SAMPLE_CHUNKS, cr, 0,
                           (const uint64_t *)nullptr);
        launch_thresh(cr, nr, TOPK_SAMPLE_CHUNKS, k, thr + r0, count + r0, s);
    }
    if ((rc = check_launch(c, "ann_topk sample"))) return rc;
    TopkSink sink;
    sink.thr = thr;
    sink.count = count;
    sink.key = keys;
    sink.score = raw;
    sink.cap = (int)cap;
    if (const int nk = skinny_shape_nk(w, c->d_aq, w.Kp, true)) {
        // 128 rows a launch, whatever M (each launch reads the index once): with 256 rows'
        // accumulators the candidate epilogue spills, and at M = 1024 eight launches took
        // well under the persistent kernel's candidate pass
        for (int64_t r0 = 0; r0 < M; r0 += 128) {
            TopkSink part = sink;
            part.thr += r0;
            part.count += r0;
            part.key += r0 * cap;
            part.score += r0 * cap;
            const int64_t mr = std::min<int64_t>(128, M - r0);
            if (mr <= 32)  // one row block: the epilogue's work per score covers 32 rows, not 128
                launch_skinny_mb<1, EPI_TOPK, true>(c, w, nk, c->d_aq + r0 * w.Kp, w.Kp, c->d_as + r0, nullptr,
                                                    nullptr, 0, mr, s, part);
            else
                launch_skinny_mb<4, EPI_TOPK, true>(c, w, nk, c->d_aq + r0 * w.Kp, w.Kp, c->d_as + r0, nullptr,
                                                    nullptr, 0, mr, s, part);
        }
    } else
        launch_pt<PT_PW, EPI_TOPK, true>(c, w, c->d_aq, w.Kp, c->d_as, nullptr, nullptr, 0, M, s, sink);
    if ((rc = check_launch(c, "gemm_w8a8 topk"))) return rc;
    if (k <= TOPK_SMALL_K)
        hipLaunchKernelGGL((topk_sink_merge<TOPK_CHUNK / 256, TOPK_SMALL_K>), dim3((unsigned)M), dim3(256), 0, s,
                           (const unsigned *)count, (const uint64_t *)keys, (const float *)raw, (int)cap, (int)k,
                           hit_i, k, hit_s, k);
    else
        hipLaunchKernelGGL((topk_sink_merge<2 * TOPK_CHUNK / 256, TOPK_WIDE_K>), dim3((unsigned)M), dim3(256), 0, s,
                           (const unsigned *)count, (const uint64_t *)keys, (const float *)raw, (int)cap, (int)k,
                           hit_i, k, hit_s, k);
    return check_launch(c, "topk_sink_merge");
}

// Brings back enchip_ann_topk's results after the work enqueued on s: the hits block
// (d_hits: M k indices, M k scores, then M list sizes when count is given) in one copy,
// into the pinned staging when it fits a slot, then split into the caller's arrays.
int fetch_hits(enchip_ctx *c, hipStream_t s, int64_t M, int64_t k, int32_t *hit_index, float *hit_score,
               unsigned *count) {
    const size_t n = (size_t)(M * k) * sizeof(int32_t), bytes = 2 * n + (count ? (size_t)M * sizeof(unsigned) : 0);
    int rc;
    std::vector<char> big;
    const char *host;
    if (bytes <= kStageChunk) {
        if ((rc = ensure_stage(c))) return rc;
        for (hipEvent_t e : c->stage_ev) HIP_TRY(c, hipEventSynchronize(e));  // no DMA still reads a slot
        HIP_TRY(c, hipMemcpyAsync(c->h_stage, c->d_hits, bytes, hipMemcpyDeviceToHost, s));
        HIP_TRY(c, hipStreamSynchronize(s));
        host = c->h_stage;
    } else {
        big.resize(bytes);
        if ((rc = download(c, big.data(), c->d_hits, bytes, s))) return rc;
        HIP_TRY(c, hipStreamSynchronize(s));
        host = big.data();
    }
    std::memcpy(hit_index, host, n);
    std::memcpy(hit_score, host + n, n);
    if (count) std::memcpy(count, host + 2 * n, (size_t)M * sizeof(unsigned));
    return ENCHIP_OK;
}

}  // namespace

int enchip_topk_rows_dev(enchip_ctx *ctx, const float *d_scores, int64_t ld, int64_t rows, int64_t n, int64_t k,
                         int32_t *d_index, int64_t ldi, float *d_score, int64_t lds, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (rows < 0 || n < 0 || n > 0x7fffffff || k < 0 || k > enchip::TOPK_MAX_K || ld < n || ldi < k || lds < k)
        return fail(ctx, ENCHIP_ERR_ARG, "topk: bad shape rows=%lld n=%lld k=%lld (k <= %d)", (long long)rows,
                    (long long)n, (long long)k, enchip::TOPK_MAX_K);
    if (rows == 0 || k == 0) return ENCHIP_OK;
    if ((n > 0 && !d_scores) || !d_index || !d_score) return fail(ctx, ENCHIP_ERR_ARG, "topk: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    int rc;
    if ((rc = scratch_wait(ctx, s))) return rc;
    if ((rc = launch_topk(ctx, d_scores, ld, rows, n, k, d_index, ldi, d_score, lds, s))) return rc;
    return scratch_record(ctx, s);
}

int enchip_ann_topk(enchip_ctx *ctx, enchip_weight h, const float *queries, int64_t M, int64_t k, int32_t *hit_index,
                    float *hit_score) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    Weight *w;
    int rc = find_weight(ctx, h, &w);
    if (rc) return rc;
    if (M < 0 || M > ((int64_t)1 << 30) || k < 0 || k > enchip::TOPK_MAX_K || w->N > 0x7fffffff)
        return fail(ctx, ENCHIP_ERR_ARG, "ann_topk: bad shape M=%lld k=%lld (k <= %d)", (long long)M, (long long)k,
                    enchip::TOPK_MAX_K);
    if (M == 0 || k == 0) return ENCHIP_OK;
    if ((w->K > 0 && !queries) || !hit_index || !hit_score) return fail(ctx, ENCHIP_ERR_ARG, "ann_topk: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    const int64_t K = w->K, N = w->N;
    if ((rc = ensure(ctx, &ctx->d_a, &ctx->a_cap, std::max<size_t>((size_t)(M * K) * sizeof(float), 16)))) return rc;
    if ((rc = ensure(ctx, &ctx->d_hits, &ctx->hits_cap, (size_t)(2 * M * k + M) * sizeof(int32_t)))) return rc;
    int32_t *d_hit_i = ctx->d_hits;
    float *d_hit_s = reinterpret_cast<float *>(d_hit_i + M * k);
    unsigned *d_count = reinterpret_cast<unsigned *>(d_hit_s + M * k);
    if ((rc = ensure_act_scratch(ctx, M, w->Kp))) return rc;
    hipStream_t s = ctx->stream;
    if ((rc = scratch_wait(ctx, s))) return rc;
    if ((rc = upload(ctx, ctx->d_a, queries, (size_t)(M * K) * sizeof(float), s))) return rc;
    // the bias-free W8A8 scores (ann/backend.go:25-29), then the selection on the device
    // (d_dst, from the context allocator, is 256-byte aligned: the route does not depend
    // on whether it is allocated yet)
    const bool fuse = ann_fused_ok(ctx, *w, M, k, route_af(ctx, *w, M, nullptr, N));
    const bool af = fuse || route_af(ctx, *w, M, nullptr, N);  // the codes' layout, for both routes
    if ((rc = launch_quant(ctx, ctx->d_a, M, K, ctx->d_aq, w->Kp, ctx->d_as, s, af))) return rc;
    if (fuse) {
        if ((rc = launch_ann_fused(ctx, *w, M, k, s, d_hit_i, d_hit_s, d_count))) return rc;
        if ((rc = scratch_record(ctx, s))) return rc;
        std::vector<unsigned> count((size_t)M);
        if ((rc = fetch_hits(ctx, s, M, k, hit_index, hit_score, count.data()))) return rc;
        ++ctx->ann_fused_calls;
        if (*std::max_element(count.begin(), count.end()) <= (unsigned)sink_cap(k)) return ENCHIP_OK;
        ++ctx->ann_fallbacks;  // some row's list overflowed: the two-pass route below
    }
    if ((rc = ensure(ctx, &ctx->d_dst, &ctx->dst_cap, (size_t)(M * N) * sizeof(float)))) return rc;
    if ((rc = launch_gemm(ctx, *w, ctx->d_aq, w->Kp, ctx->d_as, nullptr, enchip::EPI_F32, ctx->d_dst, N, M, s, af)))
        return rc;
    if ((rc = launch_topk(ctx, ctx->d_dst, N, M, N, k, d_hit_i, k, d_hit_s, k, s))) return rc;
    if ((rc = scratch_record(ctx, s))) return rc;
    return fetch_hits(ctx, s, M, k, hit_index, hit_score, nullptr);
}

int enchip_ann_topk_stats(enchip_ctx *ctx, int64_t *fused, int64_t *fallbacks) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (!fused || !fallbacks) return fail(ctx, ENCHIP_ERR_ARG, "ann_topk_stats: null pointer");
    *fused = ctx->ann_fused_calls;
    *fallbacks = ctx->ann_fallbacks;
    return ENCHIP_OK;
}

int enchip_embed_rows_dev(enchip_ctx *ctx, const int32_t *d_ids, const int32_t *d_segs, int64_t nseq, int64_t L,
                          const float *d_word, int64_t vocab, const float *d_pos, int64_t npos, int64_t pos_off,
                          const float *d_type, int64_t type_vocab, int64_t D, float *d_h, int64_t ldh,
                          void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (nseq < 0 || L < 0 || D <= 0 || ldh < D || vocab <= 0 || pos_off < 0 || type_vocab < 0 ||
        L + pos_off > npos || nseq * L > ((int64_t)1 << 31) || D > ((int64_t)1 << 20))
        return fail(ctx, ENCHIP_ERR_ARG,
                    "embed: bad shape nseq=%lld L=%lld D=%lld ldh=%lld vocab=%lld npos=%lld pos_off=%lld "
                    "type_vocab=%lld (positions L + pos_off must be < npos rows)",
                    (long long)nseq, (long long)L, (long long)D, (long long)ldh, (long long)vocab, (long long)npos,
                    (long long)pos_off, (long long)type_vocab);
    if (nseq == 0 || L == 0) return ENCHIP_OK;
    if (!d_ids || !d_word || !d_pos || !d_h || (type_vocab > 0 && !d_type))
        return fail(ctx, ENCHIP_ERR_ARG, "embed: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    const bool vec = D % 4 == 0 && ldh % 4 == 0 && (uintptr_t)d_word % 16 == 0 && (uintptr_t)d_pos % 16 == 0 &&
                     (uintptr_t)d_type % 16 == 0 && (uintptr_t)d_h % 16 == 0;
    // whole sequences per launch, at most about kRowChunk rows (a row's position is its
    // index within the launch modulo L)
    const int64_t zchunk = std::max<int64_t>(1, kRowChunk / L);
    for (int64_t z0 = 0; z0 < nseq; z0 += zchunk) {
        const int64_t r0 = z0 * L, rows = std::min(zchunk, nseq - z0) * L;
        const dim3 grid((unsigned)((rows + 3) / 4));
        const int32_t *segs = d_segs ? d_segs + r0 : nullptr;
        if (vec)
            hipLaunchKernelGGL(enchip::embed_rows<true>, grid, dim3(256), 0, s, d_ids + r0, segs, rows, (int)L, d_word,
                               vocab, d_pos, (int)pos_off, d_type, type_vocab, (int)D, d_h + r0 * ldh, ldh);
        else
            hipLaunchKernelGGL(enchip::embed_rows<false>, grid, dim3(256), 0, s, d_ids + r0, segs, rows, (int)L, d_word,
                               vocab, d_pos, (int)pos_off, d_type, type_vocab, (int)D, d_h + r0 * ldh, ldh);
    }
    return check_launch(ctx, "embed_rows");
}

int enchip_bias_act_rows_dev(enchip_ctx *ctx, float *d_x, int64_t ld, int64_t rows, int64_t cols,
                             const float *d_bias, int act, void *stream) {
    if (!ctx) return ENCHIP_ERR_ARG;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (act != ENCHIP_ACT_NONE && act != ENCHIP_ACT_TANH)
        return fail(ctx, ENCHIP_ERR_ARG, "bias_act: act must be ENCHIP_ACT_NONE or ENCHIP_ACT_TANH, got %d", act);
    if (rows < 0 || cols < 0 || ld < cols || cols > ((int64_t)1 << 30))
        return fail(ctx, ENCHIP_ERR_ARG, "bias_act: bad shape rows=%lld cols=%lld ld=%lld", (long long)rows,
                    (long long)cols, (long long)ld);
    if (rows == 0 || cols == 0) return ENCHIP_OK;
    if (!d_x) return fail(ctx, ENCHIP_ERR_ARG, "bias_act: null pointer");
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    // whole rows per launch, at most 2^30 elements (one thread each)
    const int64_t rchunk = std::max<int64_t>(1, ((int64_t)1 << 30) / cols);
    for (int64_t r0 = 0; r0 < rows; r0 += rchunk) {
        const int64_t n = std::min(rchunk, rows - r0);
        const dim3 grid((unsigned)((n * cols + 255) / 256));
        if (act == ENCHIP_ACT_TANH)
            hipLaunchKernelGGL(enchip::bias_act_rows<true>, grid, dim3(256), 0, s, d_x + r0 * ld, ld, n, (int)cols,
                               d_bias);
        else
            hipLaunchKernelGGL(enchip::bias_act_rows<false>, grid, dim3(256), 0, s, d_x + r0 * ld, ld, n, (int)cols,
                               d_bias);
    }
    return check_launch(ctx, "bias_act_rows");
}
