// C-ABI entry points of libctattn.so (declared in include/ctattn.h).
//
// Validates arguments on the host before any HIP call, picks the kernel family, launches
// on the caller's stream and turns failures into (hipError_t, message) pairs.  With the
// environment variable CTATTN_SYNC_CHECK=1 every entry point also synchronises the stream
// and reports asynchronous kernel errors (debug mode; off by default).
#include "attn_launch.h"
#include "capi_util.h"
#include "ctattn.h"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <mutex>

namespace ctattn {
namespace capi {

thread_local char g_err[512] = {0};

int fail(hipError_t code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return int(code);
}

int ok() {
    g_err[0] = '\0';
    return 0;
}

bool sync_check_enabled() {
    static const bool on = [] {
        const char *e = std::getenv("CTATTN_SYNC_CHECK");
        return e != nullptr && e[0] == '1';
    }();
    return on;
}

int finish(const char *fn, hipError_t e, hipStream_t stream) {
    if (e != hipSuccess)
        return fail(e, "%s: kernel launch failed: %s", fn, hipGetErrorString(e));
    if (sync_check_enabled()) {
        e = hipStreamSynchronize(stream);
        if (e == hipSuccess) e = hipGetLastError();
        if (e != hipSuccess)
            return fail(e, "%s: kernel execution failed: %s", fn, hipGetErrorString(e));
    }
    return ok();
}

int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

}  // namespace capi
}  // namespace ctattn

namespace {

using ctattn::capi::align_up;
using ctattn::capi::fail;
using ctattn::capi::finish;
using ctattn::capi::ok;

std::atomic<int> g_policy{CTATTN_POLICY_AUTO};

// Validates dtype and sizes; returns 0 or an error code (message set).
int validate_shape(const char *fn, int dtype, int64_t B, int64_t H, int64_t T, int64_t d) {
    if (dtype != CTATTN_F32 && dtype != CTATTN_BF16 && dtype != CTATTN_F16 && dtype != CTATTN_F64)
        return fail(hipErrorInvalidValue, "%s: unknown dtype %d (0 = f32, 1 = bf16, 2 = f16, 3 = f64)", fn,
                    dtype);
    if (B < 0 || H < 0 || T < 0)
        return fail(hipErrorInvalidValue, "%s: negative size B=%lld H=%lld T=%lld", fn,
                    (long long)B, (long long)H, (long long)T);
    if (d < 1 || d > 256)
        return fail(hipErrorNotSupported, "%s: head dim d=%lld unsupported (1 <= d <= 256)", fn,
                    (long long)d);
    // B*H*T must fit a 1-D grid of rows, and B*H*T*d an int64 element offset.
    const double rows = double(B) * double(H) * double(T);
    if (rows > 2147483647.0)
        return fail(hipErrorInvalidValue, "%s: B*H*T = %.0f exceeds 2^31-1", fn, rows);
    return 0;
}

// fp32, bf16 and fp16 storage: the fp32-accumulating MFMA kernels (fp32 LSE / delta).
bool use_mfma_fwd(int dtype, int64_t d) {
    return (dtype == CTATTN_F32 || dtype == CTATTN_BF16 || dtype == CTATTN_F16) && g_policy.load() != CTATTN_POLICY_GENERIC &&
           ctattn::mfma_fwd_supported(dtype, d);
}
bool use_mfma_bwd(int dtype, int64_t d) {
    return (dtype == CTATTN_F32 || dtype == CTATTN_BF16 || dtype == CTATTN_F16) && g_policy.load() != CTATTN_POLICY_GENERIC &&
           ctattn::mfma_bwd_supported(dtype, d);
}
// fp64 storage: the fp64 MFMA kernels (fp64 LSE / delta, no scratch beyond delta).
bool use_f64_mfma(int dtype, int64_t d) {
    return dtype == CTATTN_F64 && g_policy.load() != CTATTN_POLICY_GENERIC && ctattn::f64_mfma_supported(d);
}
// The MFMA kernels move 16 bytes per load (float4 / double2 / direct-to-LDS dwordx4); row
// strides are multiples of 16 bytes for d in {32, 64, 128}, so 16-byte-aligned base pointers
// suffice.  Element-aligned views that are not (a tensor offset into its storage) take the
// generic kernels, which access element by element.
bool aligned16(std::initializer_list<const void *> ps) {
    for (const void *p : ps)
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
    return true;
}
// Bytes of one LSE / delta element: fp64 for fp64 storage, fp32 otherwise.
int64_t stat_bytes(int dtype) { return dtype == CTATTN_F64 ? 8 : 4; }
bool deterministic_policy() { return g_policy.load() == CTATTN_POLICY_DETERMINISTIC; }

// Bytes of one storage element.
int64_t elem_bytes(int dtype) { return dtype == CTATTN_F64 ? 8 : dtype == CTATTN_F32 ? 4 : 2; }

// Head dims up to 128 without an MFMA kernel of their own (not 32, 64 or 128) run the MFMA
// kernels of the next width on zero-padded copies of the tensors (attn_pad.hip), with the
// scores scaled by 1 / sqrt(d) of the real head dim: that width, or 0 when d takes its own
// MFMA kernels, is above 128, or the policy asks for the generic kernels.
int64_t padded_width(int dtype, int64_t d) {
    if (g_policy.load() == CTATTN_POLICY_GENERIC || d > 128) return 0;
    const int64_t dp = d <= 32 ? 32 : d <= 64 ? 64 : 128;
    if (dp == d) return 0;
    const bool mfma = dtype == CTATTN_F64 ? ctattn::f64_mfma_supported(dp)
                                          : ctattn::mfma_fwd_supported(dtype, dp) && ctattn::mfma_bwd_supported(dtype, dp);
    return mfma ? dp : 0;
}
// The shape the MFMA kernels see for padded width dp.
ctattn::AttnShape padded_shape(const ctattn::AttnShape &s, int64_t dp) {
    ctattn::AttnShape sp = s;
    sp.d = dp;
    sp.scale_d = s.d;
    return sp;
}
// Backward workspace of the padded path: the MFMA backward's own (delta and friends, for the
// padded shape) followed by the eight padded copies q, k, v, o, dO, dQ, dK, dV.
int64_t padded_copy_bytes(int dtype, const ctattn::AttnShape &s, int64_t dp) {
    return align_up(s.rows() * dp * elem_bytes(dtype));
}

// ---- Scratch of ctattn_bwd_noalloc: the backward workspace (delta and friends) in a
// file-scope device array instead of caller- or library-allocated memory.  Every GPU the
// library runs on holds its own copy until the process ends; all calls on one GPU share it.
// `scratch` names a host-side stand-in in host code: kernels receive the device address that
// hipGetSymbolAddress returns for the stream's device, looked up once per device.
static_assert(CTATTN_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");
__device__ __align__(256) unsigned char scratch[CTATTN_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device that owns `stream` (the current device for the
// null stream).  Returns 0 or an error code (message set).
int scratch_for_stream(hipStream_t stream, void **out) {
    int dev = 0;
    hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess)
        return fail(e, "ctattn_bwd_noalloc: cannot find the stream's device: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(hipErrorInvalidDevice, "ctattn_bwd_noalloc: device %d beyond the %d supported", dev,
                    kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        int cur = 0;
        e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        void *p = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) {
            const hipError_t e2 = hipSetDevice(cur);
            if (e == hipSuccess) e = e2;
        }
        if (e != hipSuccess || p == nullptr)
            return fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                        "ctattn_bwd_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

// Backward workspace bytes: delta = rowsum(dO * O), [B, H, T] (fp64 for fp64 storage, else
// fp32), always first; then the MFMA backward's scratch (with_ds: including the bf16 / fp16 dS
// tiles, which a smaller workspace leaves out); for a padded head dim, the padded shape's
// scratch and the eight padded copies.
int64_t bwd_workspace_bytes(int dtype, const ctattn::AttnShape &s, bool with_ds) {
    int64_t bytes = align_up(s.rows() * stat_bytes(dtype));
    if (const int64_t dp = padded_width(dtype, s.d)) {
        if (dtype != CTATTN_F64)
            bytes += align_up(ctattn::mfma_bwd_workspace_bytes(dtype, padded_shape(s, dp), deterministic_policy(), with_ds));
        bytes += 8 * padded_copy_bytes(dtype, s, dp);
    } else if (use_mfma_bwd(dtype, s.d)) {
        bytes += align_up(ctattn::mfma_bwd_workspace_bytes(dtype, s, deterministic_policy(), with_ds));
    }
    return bytes;
}

// Stream-ordered memory for the forward's padded copies (ctattn_fwd takes no workspace): a
// pool per device owned by the library.  Up to kPoolKeepBytes of freed memory stay in the
// pool across synchronisations, so later calls reuse it without going back to the driver;
// beyond that (very large problems) the pool returns memory at the next synchronisation.
constexpr uint64_t kPoolKeepBytes = uint64_t(1) << 30;
std::mutex g_pool_mutex;
hipMemPool_t g_pool[kMaxDevices] = {};

int pool_for_stream(hipStream_t stream, hipMemPool_t *out) {
    int dev = 0;
    hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return fail(e, "ctattn_fwd: cannot find the stream's device: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(hipErrorInvalidDevice, "ctattn_fwd: device %d beyond the %d supported", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    if (g_pool[dev] == nullptr) {
        hipMemPoolProps props = {};
        props.allocType = hipMemAllocationTypePinned;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = dev;
        hipMemPool_t pool = nullptr;
        e = hipMemPoolCreate(&pool, &props);
        if (e == hipSuccess) {
            uint64_t keep = kPoolKeepBytes;
            e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
            if (e != hipSuccess) (void)hipMemPoolDestroy(pool);
        }
        if (e != hipSuccess)
            return fail(e, "ctattn_fwd: cannot create the memory pool of device %d: %s", dev, hipGetErrorString(e));
        g_pool[dev] = pool;
    }
    *out = g_pool[dev];
    return 0;
}

// The forward for a head dim that runs on the MFMA kernels of width dp: q, k, v padded into
// buf (4 padded copies: q, k, v, o), the kernels writing O into a padded buffer (LSE straight
// into the caller's, whose layout does not depend on d), O copied back.
hipError_t fwd_padded_in(int dtype, int64_t dp, const void *q, const void *k, const void *v, void *o, void *lse,
                         const ctattn::AttnShape &s, hipStream_t st, void *buf) {
    const int eb = int(elem_bytes(dtype));
    const int64_t rows = s.rows();
    const int64_t tb = padded_copy_bytes(dtype, s, dp);
    char *p = static_cast<char *>(buf);
    void *qp = p, *kp = p + tb, *vp = p + 2 * tb, *op = p + 3 * tb;
    const ctattn::AttnShape sp = padded_shape(s, dp);
    const int d = int(s.d), w = int(dp);
    const void *in[3] = {q, k, v};
    void *padded[3] = {qp, kp, vp};
    hipError_t e = ctattn::launch_pad_rows(eb, in, padded, 3, rows, d, w, st);
    if (e == hipSuccess)
        e = dtype == CTATTN_F64 ? ctattn::launch_f64_fwd(qp, kp, vp, op, lse, sp, st)
                                : ctattn::launch_mfma_fwd(dtype, qp, kp, vp, op, static_cast<float *>(lse), sp, st);
    const void *po[1] = {op};
    void *oo[1] = {o};
    if (e == hipSuccess) e = ctattn::launch_unpad_rows(eb, po, oo, 1, rows, d, w, st);
    return e;
}

// ctattn_fwd's padded path: the copies in stream-ordered memory from the library's pool.
int fwd_padded_pool(int dtype, int64_t dp, const void *q, const void *k, const void *v, void *o, void *lse,
                    const ctattn::AttnShape &s, hipStream_t st) {
    const int64_t bytes = 4 * padded_copy_bytes(dtype, s, dp);
    hipMemPool_t pool = nullptr;
    if (int rc = pool_for_stream(st, &pool)) return rc;
    void *buf = nullptr;
    hipError_t e = hipMallocFromPoolAsync(&buf, size_t(bytes), pool, st);
    if (e != hipSuccess)
        return fail(e, "ctattn_fwd: %lld bytes for the head dim %lld -> %lld copies: %s", (long long)bytes,
                    (long long)s.d, (long long)dp, hipGetErrorString(e));
    e = fwd_padded_in(dtype, dp, q, k, v, o, lse, s, st, buf);
    const hipError_t ef = hipFreeAsync(buf, st);  // after every use of buf on the stream
    return finish("ctattn_fwd", e != hipSuccess ? e : ef, st);
}

// The bf16 / fp16 dS tiles go into the default backward workspace only while they take no
// more than twice the bytes of q, k and v together, so that workspace stays linear in
// B * H * T; ctattn_bwd_workspace_bytes_max always includes them.
bool ds_in_default(int dtype, const ctattn::AttnShape &s) {
    const int64_t ds = bwd_workspace_bytes(dtype, s, true) - bwd_workspace_bytes(dtype, s, false);
    return ds <= 2 * 3 * s.rows() * s.d * elem_bytes(dtype);
}

}  // namespace

extern "C" {

int ctattn_fwd(int dtype, const void *q, const void *k, const void *v, void *o, void *lse,
               int64_t B, int64_t H, int64_t T, int64_t d, int causal, void *stream) {
    if (int rc = validate_shape("ctattn_fwd", dtype, B, H, T, d)) return rc;
    const ctattn::AttnShape s{B, H, T, d, causal != 0};
    if (s.rows() == 0) return ok();
    if (!q || !k || !v || !o)
        return fail(hipErrorInvalidValue, "ctattn_fwd: null q/k/v/o pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (const int64_t dp = padded_width(dtype, d)) return fwd_padded_pool(dtype, dp, q, k, v, o, lse, s, st);
    const bool al = aligned16({q, k, v, o, lse});
    hipError_t e = use_mfma_fwd(dtype, d) && al ? ctattn::launch_mfma_fwd(dtype, q, k, v, o, static_cast<float *>(lse), s, st)
                   : use_f64_mfma(dtype, d) && al ? ctattn::launch_f64_fwd(q, k, v, o, lse, s, st)
                                                  : ctattn::launch_generic_fwd(dtype, q, k, v, o, lse, s, st);
    return finish("ctattn_fwd", e, st);
}

int64_t ctattn_fwd_workspace_bytes(int dtype, int64_t B, int64_t H, int64_t T, int64_t d) {
    if (validate_shape("ctattn_fwd_workspace_bytes", dtype, B, H, T, d)) return -1;
    ok();
    const ctattn::AttnShape s{B, H, T, d, false};
    const int64_t dp = padded_width(dtype, d);
    return dp != 0 ? 4 * padded_copy_bytes(dtype, s, dp) : 0;
}

int ctattn_fwd_ws(int dtype, const void *q, const void *k, const void *v, void *o, void *lse, void *workspace,
                  int64_t workspace_bytes, int64_t B, int64_t H, int64_t T, int64_t d, int causal, void *stream) {
    if (int rc = validate_shape("ctattn_fwd_ws", dtype, B, H, T, d)) return rc;
    const ctattn::AttnShape s{B, H, T, d, causal != 0};
    if (s.rows() == 0) return ok();
    const int64_t dp = padded_width(dtype, d);
    if (dp == 0) return ctattn_fwd(dtype, q, k, v, o, lse, B, H, T, d, causal, stream);
    if (!q || !k || !v || !o) return fail(hipErrorInvalidValue, "ctattn_fwd_ws: null q/k/v/o pointer");
    const int64_t need = 4 * padded_copy_bytes(dtype, s, dp);
    if (workspace == nullptr || workspace_bytes < need || !aligned16({workspace}))
        return fail(hipErrorInvalidValue,
                    "ctattn_fwd_ws: a 16-byte aligned workspace of %lld bytes is needed "
                    "(ctattn_fwd_workspace_bytes), %lld given",
                    (long long)need, (long long)workspace_bytes);
    hipStream_t st = static_cast<hipStream_t>(stream);
    return finish("ctattn_fwd_ws", fwd_padded_in(dtype, dp, q, k, v, o, lse, s, st, workspace), st);
}

int64_t ctattn_bwd_workspace_bytes(int dtype, int64_t B, int64_t H, int64_t T, int64_t d,
                                   int causal) {
    if (validate_shape("ctattn_bwd_workspace_bytes", dtype, B, H, T, d)) return -1;
    ok();
    const ctattn::AttnShape s{B, H, T, d, causal != 0};
    return bwd_workspace_bytes(dtype, s, ds_in_default(dtype, s));
}

int64_t ctattn_bwd_workspace_bytes_max(int dtype, int64_t B, int64_t H, int64_t T, int64_t d,
                                       int causal) {
    if (validate_shape("ctattn_bwd_workspace_bytes_max", dtype, B, H, T, d)) return -1;
    ok();
    return bwd_workspace_bytes(dtype, ctattn::AttnShape{B, H, T, d, causal != 0}, true);
}

int ctattn_bwd(int dtype, const void *q, const void *k, const void *v, const void *o,
               const void *dout, const void *lse, void *dq, void *dk, void *dv,
               void *workspace, int64_t workspace_bytes, int64_t B, int64_t H, int64_t T,
               int64_t d, int causal, void *stream) {
    if (int rc = validate_shape("ctattn_bwd", dtype, B, H, T, d)) return rc;
    const ctattn::AttnShape s{B, H, T, d, causal != 0};
    if (s.rows() == 0) return ok();
    if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv)
        return fail(hipErrorInvalidValue, "ctattn_bwd: null tensor pointer");
    // Any workspace from `need` (no bf16 / fp16 dS tiles) up works; the dS tiles are used when
    // it holds them (ctattn_bwd_workspace_bytes_max).
    const int64_t need = bwd_workspace_bytes(dtype, s, false);
    if (workspace == nullptr || workspace_bytes < need)
        return fail(hipErrorInvalidValue,
                    "ctattn_bwd: workspace of %lld bytes given, %lld needed "
                    "(ctattn_bwd_workspace_bytes)",
                    (long long)workspace_bytes, (long long)need);
    const bool with_ds = workspace_bytes >= bwd_workspace_bytes(dtype, s, true);
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e;
    // Misaligned tensors take the generic kernels, whose workspace (delta only) is a prefix of
    // what ctattn_bwd_workspace_bytes asked for.
    const bool al = aligned16({q, k, v, o, dout, lse, dq, dk, dv, workspace});
    const int64_t dp = padded_width(dtype, d);
    if (dp != 0 && aligned16({workspace})) {
        // Head dim d on the MFMA kernels of width dp: the workspace holds delta, the padded
        // shape's MFMA scratch, then the padded q, k, v, o, dO (inputs) and dQ, dK, dV.
        const ctattn::AttnShape sp = padded_shape(s, dp);
        const int eb = int(elem_bytes(dtype));
        const int64_t rows = s.rows(), tb = padded_copy_bytes(dtype, s, dp);
        char *w = static_cast<char *>(workspace);
        void *delta = w;
        w += align_up(rows * stat_bytes(dtype));
        void *extra = w;
        const int64_t extra_bytes =
            dtype != CTATTN_F64 ? align_up(ctattn::mfma_bwd_workspace_bytes(dtype, sp, deterministic_policy(), with_ds))
                                : 0;
        w += extra_bytes;
        void *cp[8];
        for (int i = 0; i < 8; ++i) cp[i] = w + i * tb;
        const void *in[5] = {q, k, v, o, dout};
        const int di = int(d), wi = int(dp);
        e = ctattn::launch_pad_rows(eb, in, cp, 5, rows, di, wi, st);
        if (e == hipSuccess)
            e = dtype == CTATTN_F64
                    ? ctattn::launch_f64_bwd(cp[0], cp[1], cp[2], cp[3], cp[4], lse, delta, cp[5], cp[6], cp[7], sp, st)
                    : ctattn::launch_mfma_bwd(dtype, cp[0], cp[1], cp[2], cp[3], cp[4], static_cast<const float *>(lse),
                                              static_cast<float *>(delta), cp[5], cp[6], cp[7], extra, extra_bytes,
                                              deterministic_policy(), sp, st);
        const void *grads[3] = {cp[5], cp[6], cp[7]};
        void *out[3] = {dq, dk, dv};
        if (e == hipSuccess) e = ctattn::launch_unpad_rows(eb, grads, out, 3, rows, di, wi, st);
    } else if (use_mfma_bwd(dtype, d) && al) {
        const int64_t head = align_up(s.rows() * stat_bytes(dtype));
        void *extra = static_cast<char *>(workspace) + head;
        e = ctattn::launch_mfma_bwd(dtype, q, k, v, o, dout, static_cast<const float *>(lse),
                                    static_cast<float *>(workspace), dq, dk, dv, extra, workspace_bytes - head,
                                    deterministic_policy(), s, st);
    } else if (use_f64_mfma(dtype, d) && al) {
        e = ctattn::launch_f64_bwd(q, k, v, o, dout, lse, workspace, dq, dk, dv, s, st);
    } else {
        e = ctattn::launch_generic_bwd(dtype, q, k, v, o, dout, lse, dq, dk, dv, workspace, s, st);
    }
    return finish("ctattn_bwd", e, st);
}

int ctattn_bwd_noalloc(int dtype, const void *q, const void *k, const void *v, const void *o,
                       const void *dout, const void *lse, void *dq, void *dk, void *dv, int64_t B,
                       int64_t H, int64_t T, int64_t d, int causal, void *stream) {
    if (int rc = validate_shape("ctattn_bwd_noalloc", dtype, B, H, T, d)) return rc;
    // The smallest workspace that works (the bf16 / fp16 dS tiles only when they fit too).
    const int64_t need = bwd_workspace_bytes(dtype, ctattn::AttnShape{B, H, T, d, causal != 0}, false);
    if (need > CTATTN_NOALLOC_SCRATCH_BYTES)
        return fail(hipErrorInvalidValue,
                    "ctattn_bwd_noalloc: this problem needs %lld bytes of scratch, more than the %lld of the "
                    "static scratch buffer (use ctattn_bwd with a workspace)",
                    (long long)need, (long long)CTATTN_NOALLOC_SCRATCH_BYTES);
    if ((B * H * T) == 0) return ok();
    if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv)
        return fail(hipErrorInvalidValue, "ctattn_bwd_noalloc: null tensor pointer");
    void *ws = nullptr;
    if (int rc = scratch_for_stream(static_cast<hipStream_t>(stream), &ws)) return rc;
    const int rc = ctattn_bwd(dtype, q, k, v, o, dout, lse, dq, dk, dv, ws, CTATTN_NOALLOC_SCRATCH_BYTES, B, H,
                              T, d, causal, stream);
    if (rc != 0) {
        // Keep ctattn_bwd's message, named for this entry point.
        char msg[sizeof(ctattn::capi::g_err)];
        std::snprintf(msg, sizeof(msg), "%s", ctattn::capi::g_err);
        return fail(hipError_t(rc), "ctattn_bwd_noalloc: %s", msg);
    }
    return ok();
}

const char *ctattn_last_error(void) { return ctattn::capi::g_err; }

int ctattn_set_policy(int policy) {
    if (policy != CTATTN_POLICY_AUTO && policy != CTATTN_POLICY_GENERIC &&
        policy != CTATTN_POLICY_DETERMINISTIC)
        return -1;
    return g_policy.exchange(policy);
}

int ctattn_get_policy(void) { return g_policy.load(); }

int ctattn_version(void) { return 200; }

}  // extern "C"
