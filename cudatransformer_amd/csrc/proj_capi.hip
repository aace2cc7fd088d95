// C-ABI entry points of the attention layer's projections and of the plain linear layers
// (declared in include/ctattn.h).
//
// Each entry point validates its arguments on the host, describes its products as
// separable views (row-major [B*T, E] activations, [B, H, T, d] attention tensors, [out][in]
// weights) and launches the split-K-in-workgroup MFMA GEMMs of linear_gemm.hip (fp32, bf16,
// fp16) on the caller's stream.  fp64, shapes outside that family's domain (K not a multiple
// of the K chunk, an unaligned operand, head dims that split a chunk) and the GENERIC policy
// take the projection family of proj_gemm.hip.
#include "capi_util.h"
#include "ctattn.h"
#include "linear_gemm.h"
#include "proj_launch.h"

#include <algorithm>
#include <cstdint>

namespace {

using ctattn::GemmParams;
using ctattn::head_view;
using ctattn::linear_view;
using ctattn::MatView;
using ctattn::capi::align_up;
using ctattn::capi::fail;
using ctattn::capi::finish;
using ctattn::capi::ok;

struct ProjShape {
    int64_t B, T, E, H, d;
    int64_t rows() const { return B * T; }
    int64_t hd() const { return H * d; }
};

bool known_dtype(int dtype) {
    return dtype == CTATTN_F32 || dtype == CTATTN_BF16 || dtype == CTATTN_F16 || dtype == CTATTN_F64;
}

int validate_proj(const char *fn, int dtype, const ProjShape &s) {
    if (!known_dtype(dtype))
        return fail(hipErrorInvalidValue, "%s: unknown dtype %d (0 = f32, 1 = bf16, 2 = f16, 3 = f64)", fn, dtype);
    if (s.B < 0 || s.T < 0)
        return fail(hipErrorInvalidValue, "%s: negative size B=%lld T=%lld", fn, (long long)s.B,
                    (long long)s.T);
    if (s.E < 1 || s.H < 1 || s.d < 1)
        return fail(hipErrorInvalidValue, "%s: E=%lld H=%lld d=%lld must be >= 1", fn, (long long)s.E,
                    (long long)s.H, (long long)s.d);
    // GEMM indices (rows B*T, columns E and H*d) are 32-bit in the kernels.
    const double lim = 2147483647.0;
    if (double(s.B) * double(s.T) > lim || double(s.E) > lim || double(s.H) * double(s.d) > lim)
        return fail(hipErrorInvalidValue, "%s: B*T, E and H*d must each be below 2^31", fn);
    return 0;
}

int elem_bytes(int dtype) { return dtype == CTATTN_F64 ? 8 : dtype == CTATTN_F32 ? 4 : 2; }

// 4-element vector loads need every pitch / head dim to be a multiple of 4 and every base
// pointer 4-element aligned.
bool vec4_ok(int dtype, const ProjShape &s, std::initializer_list<const void *> ptrs) {
    if (s.E % 4 != 0 || s.d % 4 != 0) return false;
    const uintptr_t a = uintptr_t(4 * elem_bytes(dtype));
    for (const void *p : ptrs)
        if (p != nullptr && uintptr_t(p) % a != 0) return false;
    return true;
}

// K splits for a small-output, long-K product (weight gradients): enough workgroups to cover
// the GPU several times, at least 16 K steps (256 k) per split.  The fp64 GEMM does not split.
int choose_splits(int dtype, int64_t M, int64_t N, int64_t K, int nbatch) {
    if (dtype == CTATTN_F64) return 1;
    const int64_t tiles = int64_t(ctattn::gemm_tile_count(M, N)) * nbatch;
    int64_t s = (1024 + tiles - 1) / tiles;
    s = std::min<int64_t>(s, std::max<int64_t>(1, ctattn::gemm_k_steps(K) / 16));
    return int(std::max<int64_t>(1, std::min<int64_t>(s, 16)));
}

int64_t splitk_bytes(int dtype, int64_t M, int64_t N, int64_t K, int nbatch) {
    const int s = choose_splits(dtype, M, N, K, nbatch);
    return s > 1 ? align_up(int64_t(s) * nbatch * M * N * int64_t(sizeof(float))) : 0;
}

GemmParams make_params(int64_t M, int64_t N, int64_t K, int beta, int splits, MatView outv, float *ws) {
    GemmParams p{};
    p.M = int32_t(M);
    p.N = int32_t(N);
    p.K = int32_t(K);
    p.beta = beta;
    p.splits = splits;
    p.outv = outv;
    p.ws = ws;
    return p;
}

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

// ---- the products on linear_gemm.hip (fp32 / bf16 / fp16; the GENERIC policy keeps every
// product on the projection family as the cross-check) ----

bool lin_policy(int dtype) {
    return (dtype == CTATTN_F32 || dtype == CTATTN_BF16 || dtype == CTATTN_F16) &&
           ctattn_get_policy() != CTATTN_POLICY_GENERIC;
}
int lin_dtype(int dtype) { return dtype == CTATTN_F32 ? 0 : dtype == CTATTN_BF16 ? 1 : 2; }

ctattn::LinGemm lin_base(int dtype, bool a_kc, bool b_kc, int64_t M, int64_t N, int64_t K, int nbatch, int nseg,
                         ctattn::LinView av, ctattn::LinView bv, ctattn::LinView cv, bool beta) {
    ctattn::LinGemm g{};
    g.dtype = lin_dtype(dtype);
    g.a_kc = a_kc;
    g.b_kc = b_kc;
    g.M = M;
    g.N = N;
    g.K = K;
    g.nbatch = nbatch;
    g.nseg = nseg;
    g.av = av;
    g.bv = bv;
    g.cv = cv;
    g.beta = beta;
    return g;
}

// The six projection products, pointers filled in by the caller (null for workspace queries):
//   QKV forward  q/k/v(r, j) = sum_i x[r][i] w[j][i] + b[j]     A = x, B = w (both [.][E]), C head-split
//   QKV dW       dw[j][i] += sum_r g(r, j) x[r][i]              A = g head-split [k][m], B = x [k][n]
//   QKV dX       dx[r][i] = sum_z sum_j g_z(r, j) w_z[j][i]     A = g head-split, B = w [k][n], 3 K segments
//   out forward  y[r][e] = sum_c attn(r, c) wo[e][c] + bo[e]    A = attn head-split, B = wo [E][HD]
//   out dW       dwo[e][c] += sum_r dy[r][e] attn(r, c)         A = dy [k][m], B = attn head-split [k][n]
//   out dX       dc(r, c) = sum_e dy[r][e] wo[e][c]             A = dy, B = wo [k][n], C head-split
ctattn::LinGemm lin_qkv_fwd(int dtype, const ProjShape &s) {
    return lin_base(dtype, true, true, s.rows(), s.hd(), s.E, 3, 1, ctattn::lin_linear(s.E), ctattn::lin_linear(s.E),
                    ctattn::lin_heads(s.T, s.H, s.d), false);
}
ctattn::LinGemm lin_qkv_dw(int dtype, const ProjShape &s) {
    return lin_base(dtype, false, false, s.hd(), s.E, s.rows(), 3, 1, ctattn::lin_heads(s.T, s.H, s.d),
                    ctattn::lin_linear(s.E), ctattn::lin_linear(s.E), true);
}
ctattn::LinGemm lin_qkv_dx(int dtype, const ProjShape &s) {
    return lin_base(dtype, true, false, s.rows(), s.E, s.hd(), 1, 3, ctattn::lin_heads(s.T, s.H, s.d),
                    ctattn::lin_linear(s.E), ctattn::lin_linear(s.E), false);
}
ctattn::LinGemm lin_out_fwd(int dtype, const ProjShape &s) {
    return lin_base(dtype, true, true, s.rows(), s.E, s.hd(), 1, 1, ctattn::lin_heads(s.T, s.H, s.d),
                    ctattn::lin_linear(s.hd()), ctattn::lin_linear(s.E), false);
}
ctattn::LinGemm lin_out_dw(int dtype, const ProjShape &s) {
    return lin_base(dtype, false, false, s.E, s.hd(), s.rows(), 1, 1, ctattn::lin_linear(s.E),
                    ctattn::lin_heads(s.T, s.H, s.d), ctattn::lin_linear(s.hd()), true);
}
ctattn::LinGemm lin_out_dx(int dtype, const ProjShape &s) {
    return lin_base(dtype, true, false, s.rows(), s.hd(), s.E, 1, 1, ctattn::lin_linear(s.E),
                    ctattn::lin_linear(s.hd()), ctattn::lin_heads(s.T, s.H, s.d), false);
}

// Split-K bytes for either family's plan of a weight gradient.
int64_t lin_split_bytes(int dtype, const ctattn::LinGemm &g) {
    return lin_policy(dtype) ? align_up(ctattn::lin_gemm_workspace_bytes(g)) : 0;
}

}  // namespace

extern "C" {

int ctattn_qkv_proj_fwd(int dtype, const void *x, const void *wq, const void *wk, const void *wv,
                        const void *bq, const void *bk, const void *bv, void *q, void *k, void *v,
                        int64_t B, int64_t T, int64_t E, int64_t H, int64_t d, void *stream) {
    const char *fn = "ctattn_qkv_proj_fwd";
    const ProjShape s{B, T, E, H, d};
    if (int rc = validate_proj(fn, dtype, s)) return rc;
    if (s.rows() == 0) return ok();
    if (!x || !wq || !wk || !wv || !q || !k || !v) return fail(hipErrorInvalidValue, "%s: null tensor pointer", fn);
    // q/k/v(r, j) = sum_i x[r][i] w[j][i] + b[j]: A = x [rows][E] (K-contiguous), B = w [HD][E]
    // (K-contiguous), out in [B, H, T, d].
    GemmParams p = make_params(s.rows(), s.hd(), E, 0, 1, head_view(nullptr, T, H, d), nullptr);
    const void *w[3] = {wq, wk, wv}, *b[3] = {bq, bk, bv};
    void *o[3] = {q, k, v};
    for (int z = 0; z < 3; ++z) {
        p.batch[z].nseg = 1;
        p.batch[z].a[0] = linear_view(x, E);
        p.batch[z].b[0] = linear_view(w[z], E);
        p.batch[z].out = o[z];
        p.batch[z].bias = b[z];
    }
    if (lin_policy(dtype)) {
        ctattn::LinGemm g = lin_qkv_fwd(dtype, s);
        for (int z = 0; z < 3; ++z) {
            g.a[z][0] = x;
            g.b[z][0] = w[z];
            g.c[z] = o[z];
            g.bias[z] = b[z];
        }
        if (ctattn::lin_gemm_supported(g))
            return finish(fn, ctattn::launch_lin_gemm(g, nullptr, 0, as_stream(stream)), as_stream(stream));
    }
    const bool v4 = vec4_ok(dtype, s, {x, wq, wk, wv, q, k, v});
    return finish(fn, ctattn::launch_proj_gemm(dtype, p, 3, true, true, v4, as_stream(stream)), as_stream(stream));
}

int64_t ctattn_qkv_proj_bwd_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t E, int64_t H, int64_t d) {
    const ProjShape s{B, T, E, H, d};
    if (validate_proj("ctattn_qkv_proj_bwd_workspace_bytes", dtype, s)) return -1;
    ok();
    return std::max(splitk_bytes(dtype, s.hd(), E, s.rows(), 3), lin_split_bytes(dtype, lin_qkv_dw(dtype, s))) +
           align_up(ctattn::colsum_workspace_bytes(dtype, s.rows(), s.hd()));
}

int ctattn_qkv_proj_bwd(int dtype, const void *x, const void *dq, const void *dk, const void *dv,
                        const void *wq, const void *wk, const void *wv, void *dwq, void *dwk, void *dwv,
                        void *dbq, void *dbk, void *dbv, void *dx, void *workspace, int64_t workspace_bytes,
                        int64_t B, int64_t T, int64_t E, int64_t H, int64_t d, void *stream) {
    const char *fn = "ctattn_qkv_proj_bwd";
    const ProjShape s{B, T, E, H, d};
    if (int rc = validate_proj(fn, dtype, s)) return rc;
    if (s.rows() == 0) return ok();
    if (!x || !dq || !dk || !dv) return fail(hipErrorInvalidValue, "%s: null x/dq/dk/dv pointer", fn);
    const bool want_dw = dwq || dwk || dwv, want_db = dbq || dbk || dbv;
    if (want_dw && !(dwq && dwk && dwv)) return fail(hipErrorInvalidValue, "%s: give all of dwq/dwk/dwv or none", fn);
    if (want_db && !(dbq && dbk && dbv)) return fail(hipErrorInvalidValue, "%s: give all of dbq/dbk/dbv or none", fn);
    if (dx && !(wq && wk && wv)) return fail(hipErrorInvalidValue, "%s: dx needs wq/wk/wv", fn);
    const int64_t need = ctattn_qkv_proj_bwd_workspace_bytes(dtype, B, T, E, H, d);
    if ((want_dw || want_db) && (workspace == nullptr || workspace_bytes < need))
        return fail(hipErrorInvalidValue,
                    "%s: workspace of %lld bytes given, %lld needed (ctattn_qkv_proj_bwd_workspace_bytes)", fn,
                    (long long)workspace_bytes, (long long)need);
    hipStream_t st = as_stream(stream);
    const bool v4 = vec4_ok(dtype, s, {x, dq, dk, dv, wq, wk, wv, dwq, dwk, dwv, dx});
    const void *g[3] = {dq, dk, dv};
    hipError_t e = hipSuccess;
    float *ws = static_cast<float *>(workspace);
    const int64_t split_bytes =
        std::max(splitk_bytes(dtype, s.hd(), E, s.rows(), 3), lin_split_bytes(dtype, lin_qkv_dw(dtype, s)));
    bool dw_done = false, dx_done = false;
    bool db_done = false;
    if (want_dw && lin_policy(dtype)) {
        // The bias gradients (column sums of dq / dk / dv) come out of the same launch.
        ctattn::LinGemm lg = lin_qkv_dw(dtype, s);
        void *o[3] = {dwq, dwk, dwv}, *ob[3] = {dbq, dbk, dbv};
        for (int z = 0; z < 3; ++z) {
            lg.a[z][0] = g[z];
            lg.b[z][0] = x;
            lg.c[z] = o[z];
            lg.db[z] = ob[z];
        }
        if (ctattn::lin_gemm_supported(lg)) {
            e = ctattn::launch_lin_gemm(lg, workspace, split_bytes, st);
            if (e != hipSuccess) return finish(fn, e, st);
            dw_done = true;
            db_done = want_db;
        }
    }
    if (dx && lin_policy(dtype)) {
        ctattn::LinGemm lg = lin_qkv_dx(dtype, s);
        const void *w[3] = {wq, wk, wv};
        for (int z = 0; z < 3; ++z) {
            lg.a[0][z] = g[z];
            lg.b[0][z] = w[z];
        }
        lg.c[0] = dx;
        if (ctattn::lin_gemm_supported(lg)) {
            e = ctattn::launch_lin_gemm(lg, nullptr, 0, st);
            if (e != hipSuccess) return finish(fn, e, st);
            dx_done = true;
        }
    }
    if (want_dw && !dw_done) {
        // dw[j][i] += sum_r g(r, j) x[r][i]: M = HD, N = E, K = rows.  A(m=j, k=r) = g stored
        // [k][m] (head-split), B(k=r, n=i) = x stored [k][n].
        const int splits = choose_splits(dtype, s.hd(), E, s.rows(), 3);
        GemmParams p = make_params(s.hd(), E, s.rows(), 1, splits, linear_view(nullptr, E), ws);
        void *o[3] = {dwq, dwk, dwv};
        for (int z = 0; z < 3; ++z) {
            p.batch[z].nseg = 1;
            p.batch[z].a[0] = head_view(g[z], T, H, d);
            p.batch[z].b[0] = linear_view(x, E);
            p.batch[z].out = o[z];
            p.batch[z].bias = nullptr;
        }
        e = ctattn::launch_proj_gemm(dtype, p, 3, false, false, v4, st);
        if (e != hipSuccess) return finish(fn, e, st);
    }
    if (want_db && !db_done) {
        void *cws = static_cast<char *>(workspace) + split_bytes;
        void *o[3] = {dbq, dbk, dbv};
        for (int z = 0; z < 3 && e == hipSuccess; ++z)
            e = ctattn::launch_colsum_add(dtype, head_view(g[z], T, H, d), int(s.rows()), int(s.hd()), o[z], cws, st);
        if (e != hipSuccess) return finish(fn, e, st);
    }
    if (dx && !dx_done) {
        // dx[r][i] = sum_z sum_j g_z(r, j) w_z[j][i]: A = g (head-split, K-contiguous), B = w
        // stored [k][n]; three K segments into one output.
        GemmParams p = make_params(s.rows(), E, s.hd(), 0, 1, linear_view(nullptr, E), nullptr);
        const void *w[3] = {wq, wk, wv};
        p.batch[0].nseg = 3;
        for (int z = 0; z < 3; ++z) {
            p.batch[0].a[z] = head_view(g[z], T, H, d);
            p.batch[0].b[z] = linear_view(w[z], E);
        }
        p.batch[0].out = dx;
        p.batch[0].bias = nullptr;
        e = ctattn::launch_proj_gemm(dtype, p, 1, true, false, v4, st);
    }
    return finish(fn, e, st);
}

int ctattn_out_proj_fwd(int dtype, const void *c, const void *wo, const void *bo, void *y, int64_t B,
                        int64_t T, int64_t E, int64_t H, int64_t d, void *stream) {
    const char *fn = "ctattn_out_proj_fwd";
    const ProjShape s{B, T, E, H, d};
    if (int rc = validate_proj(fn, dtype, s)) return rc;
    if (s.rows() == 0) return ok();
    if (!c || !wo || !y) return fail(hipErrorInvalidValue, "%s: null tensor pointer", fn);
    // y[r][e] = sum_c attn(r, c) wo[e][c] + bo[e]: A = attention output (head-split,
    // K-contiguous), B = wo [E][HD] (K-contiguous).
    GemmParams p = make_params(s.rows(), E, s.hd(), 0, 1, linear_view(nullptr, E), nullptr);
    p.batch[0].nseg = 1;
    p.batch[0].a[0] = head_view(c, T, H, d);
    p.batch[0].b[0] = linear_view(wo, s.hd());
    p.batch[0].out = y;
    p.batch[0].bias = bo;
    if (lin_policy(dtype)) {
        ctattn::LinGemm g = lin_out_fwd(dtype, s);
        g.a[0][0] = c;
        g.b[0][0] = wo;
        g.c[0] = y;
        g.bias[0] = bo;
        if (ctattn::lin_gemm_supported(g))
            return finish(fn, ctattn::launch_lin_gemm(g, nullptr, 0, as_stream(stream)), as_stream(stream));
    }
    const bool v4 = vec4_ok(dtype, s, {c, wo, y});
    return finish(fn, ctattn::launch_proj_gemm(dtype, p, 1, true, true, v4, as_stream(stream)), as_stream(stream));
}

int64_t ctattn_out_proj_bwd_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t E, int64_t H, int64_t d) {
    const ProjShape s{B, T, E, H, d};
    if (validate_proj("ctattn_out_proj_bwd_workspace_bytes", dtype, s)) return -1;
    ok();
    return std::max(splitk_bytes(dtype, E, s.hd(), s.rows(), 1), lin_split_bytes(dtype, lin_out_dw(dtype, s))) +
           align_up(ctattn::colsum_workspace_bytes(dtype, s.rows(), E));
}

int ctattn_out_proj_bwd(int dtype, const void *c, const void *dy, const void *wo, void *dwo, void *dbo,
                        void *dc, void *workspace, int64_t workspace_bytes, int64_t B, int64_t T, int64_t E,
                        int64_t H, int64_t d, void *stream) {
    const char *fn = "ctattn_out_proj_bwd";
    const ProjShape s{B, T, E, H, d};
    if (int rc = validate_proj(fn, dtype, s)) return rc;
    if (s.rows() == 0) return ok();
    if (!dy) return fail(hipErrorInvalidValue, "%s: null dy pointer", fn);
    if (dwo && !c) return fail(hipErrorInvalidValue, "%s: dwo needs the attention output c", fn);
    if (dc && !wo) return fail(hipErrorInvalidValue, "%s: dc needs wo", fn);
    const int64_t need = ctattn_out_proj_bwd_workspace_bytes(dtype, B, T, E, H, d);
    if ((dwo || dbo) && (workspace == nullptr || workspace_bytes < need))
        return fail(hipErrorInvalidValue,
                    "%s: workspace of %lld bytes given, %lld needed (ctattn_out_proj_bwd_workspace_bytes)", fn,
                    (long long)workspace_bytes, (long long)need);
    hipStream_t st = as_stream(stream);
    const bool v4 = vec4_ok(dtype, s, {c, dy, wo, dwo, dc});
    float *ws = static_cast<float *>(workspace);
    hipError_t e = hipSuccess;
    const int64_t split_bytes =
        std::max(splitk_bytes(dtype, E, s.hd(), s.rows(), 1), lin_split_bytes(dtype, lin_out_dw(dtype, s)));
    if (dwo && lin_policy(dtype)) {
        ctattn::LinGemm g = lin_out_dw(dtype, s);
        g.a[0][0] = dy;
        g.b[0][0] = c;
        g.c[0] = dwo;
        g.db[0] = dbo;  // the bias gradient (column sums of dy) from the same launch
        if (ctattn::lin_gemm_supported(g)) {
            e = ctattn::launch_lin_gemm(g, workspace, split_bytes, st);
            if (e != hipSuccess) return finish(fn, e, st);
            dwo = nullptr;
            dbo = nullptr;
        }
    }
    if (dwo) {
        // dwo[e][c] += sum_r dy[r][e] attn(r, c): M = E, N = HD, K = rows.  A(m=e, k=r) = dy
        // stored [k][m]; B(k=r, n=c) = attention output stored [k][n] (head-split).
        const int splits = choose_splits(dtype, E, s.hd(), s.rows(), 1);
        GemmParams p = make_params(E, s.hd(), s.rows(), 1, splits, linear_view(nullptr, s.hd()), ws);
        p.batch[0].nseg = 1;
        p.batch[0].a[0] = linear_view(dy, E);
        p.batch[0].b[0] = head_view(c, T, H, d);
        p.batch[0].out = dwo;
        p.batch[0].bias = nullptr;
        e = ctattn::launch_proj_gemm(dtype, p, 1, false, false, v4, st);
        if (e != hipSuccess) return finish(fn, e, st);
    }
    if (dbo) {
        void *cws = static_cast<char *>(workspace) + split_bytes;
        e = ctattn::launch_colsum_add(dtype, linear_view(dy, E), int(s.rows()), int(E), dbo, cws, st);
        if (e != hipSuccess) return finish(fn, e, st);
    }
    if (dc && lin_policy(dtype)) {
        ctattn::LinGemm g = lin_out_dx(dtype, s);
        g.a[0][0] = dy;
        g.b[0][0] = wo;
        g.c[0] = dc;
        if (ctattn::lin_gemm_supported(g)) return finish(fn, ctattn::launch_lin_gemm(g, nullptr, 0, st), st);
    }
    if (dc) {
        // dc(r, c) = sum_e dy[r][e] wo[e][c]: A = dy (K-contiguous), B = wo stored [k][n]; out
        // in [B, H, T, d].
        GemmParams p = make_params(s.rows(), s.hd(), E, 0, 1, head_view(nullptr, T, H, d), nullptr);
        p.batch[0].nseg = 1;
        p.batch[0].a[0] = linear_view(dy, E);
        p.batch[0].b[0] = linear_view(wo, s.hd());
        p.batch[0].out = dc;
        p.batch[0].bias = nullptr;
        e = ctattn::launch_proj_gemm(dtype, p, 1, true, false, v4, st);
    }
    return finish(fn, e, st);
}

// ---- plain linear layers (LinearLayer.cu / linear_kernels.cu; also the un-embedding) ----

namespace {

int validate_linear(const char *fn, int dtype, int64_t M, int64_t N, int64_t K) {
    if (!known_dtype(dtype))
        return fail(hipErrorInvalidValue, "%s: unknown dtype %d (0 = f32, 1 = bf16, 2 = f16, 3 = f64)", fn, dtype);
    if (M < 0 || N < 1 || K < 1)
        return fail(hipErrorInvalidValue, "%s: need M >= 0, N >= 1, K >= 1 (got %lld, %lld, %lld)", fn, (long long)M,
                    (long long)N, (long long)K);
    if (M > 2147483647 || N > 2147483647 || K > 2147483647)
        return fail(hipErrorInvalidValue, "%s: M, N and K must each be below 2^31", fn);
    return 0;
}

// The linear layers' products on linear_gemm.hip (fp32 / bf16 / fp16, unless the policy asks
// for the projection family as a cross-check):
//   forward  y[m][n] = sum_k x[m][k] w[n][k] + b[n]   A = x [M][K], B = w [N][K]
//   dX       dx[m][k] = sum_n dy[m][n] w[n][k]       A = dy [M][N], B = w stored [n][k]
//   dW       dw[n][k] += sum_m dy[m][n] x[m][k]      A = dy stored [m][n], B = x stored [m][k]
ctattn::LinGemm lin_fwd(int dtype, const void *x, const void *w, const void *b, void *y, int64_t M, int64_t N,
                        int64_t K) {
    return ctattn::lin_plain(lin_dtype(dtype), true, true, M, N, K, x, K, w, K, y, N, b, false);
}
ctattn::LinGemm lin_dx(int dtype, const void *dy, const void *w, void *dx, int64_t M, int64_t N, int64_t K) {
    return ctattn::lin_plain(lin_dtype(dtype), true, false, M, K, N, dy, N, w, K, dx, K, nullptr, false);
}
ctattn::LinGemm lin_dw(int dtype, const void *x, const void *dy, void *dw, int64_t M, int64_t N, int64_t K) {
    return ctattn::lin_plain(lin_dtype(dtype), false, false, N, K, M, dy, N, x, K, dw, K, nullptr, true);
}

// Split-K partials of the weight gradient: room for either GEMM family's plan.
int64_t linear_split_bytes(int dtype, int64_t M, int64_t N, int64_t K) {
    return std::max(splitk_bytes(dtype, N, K, M, 1), lin_split_bytes(dtype, lin_dw(dtype, nullptr, nullptr, nullptr, M, N, K)));
}

bool linear_vec4(int dtype, int64_t M, int64_t N, int64_t K, std::initializer_list<const void *> ptrs) {
    if (M % 4 != 0 || N % 4 != 0 || K % 4 != 0) return false;
    const uintptr_t a = uintptr_t(4 * elem_bytes(dtype));
    for (const void *p : ptrs)
        if (p != nullptr && uintptr_t(p) % a != 0) return false;
    return true;
}

}  // namespace

int ctattn_linear_fwd(int dtype, const void *x, const void *w, const void *b, void *y, int64_t M, int64_t N,
                      int64_t K, void *stream) {
    const char *fn = "ctattn_linear_fwd";
    if (int rc = validate_linear(fn, dtype, M, N, K)) return rc;
    if (M == 0) return ok();
    if (!x || !w || !y) return fail(hipErrorInvalidValue, "%s: null x/w/y pointer", fn);
    if (lin_policy(dtype)) {
        const ctattn::LinGemm g = lin_fwd(dtype, x, w, b, y, M, N, K);
        if (ctattn::lin_gemm_supported(g))
            return finish(fn, ctattn::launch_lin_gemm(g, nullptr, 0, as_stream(stream)), as_stream(stream));
    }
    // y[m][n] = sum_k x[m][k] w[n][k] + b[n]: A = x [M][K], B = w [N][K], both K-contiguous.
    GemmParams p = make_params(M, N, K, 0, 1, linear_view(nullptr, N), nullptr);
    p.batch[0].nseg = 1;
    p.batch[0].a[0] = linear_view(x, K);
    p.batch[0].b[0] = linear_view(w, K);
    p.batch[0].out = y;
    p.batch[0].bias = b;
    const bool v4 = linear_vec4(dtype, M, N, K, {x, w, y});
    return finish(fn, ctattn::launch_proj_gemm(dtype, p, 1, true, true, v4, as_stream(stream)), as_stream(stream));
}

int64_t ctattn_linear_bwd_workspace_bytes(int dtype, int64_t M, int64_t N, int64_t K) {
    if (validate_linear("ctattn_linear_bwd_workspace_bytes", dtype, M, N, K)) return -1;
    ok();
    return linear_split_bytes(dtype, M, N, K) + align_up(ctattn::colsum_workspace_bytes(dtype, M, N));
}

int ctattn_linear_bwd(int dtype, const void *x, const void *w, const void *dy, void *dx, void *dw, void *db,
                      void *workspace, int64_t workspace_bytes, int64_t M, int64_t N, int64_t K, void *stream) {
    const char *fn = "ctattn_linear_bwd";
    if (int rc = validate_linear(fn, dtype, M, N, K)) return rc;
    if (M == 0) return ok();
    if (!dy) return fail(hipErrorInvalidValue, "%s: null dy pointer", fn);
    if (dw && !x) return fail(hipErrorInvalidValue, "%s: dw needs x", fn);
    if (dx && !w) return fail(hipErrorInvalidValue, "%s: dx needs w", fn);
    const int64_t need = ctattn_linear_bwd_workspace_bytes(dtype, M, N, K);
    if ((dw || db) && (workspace == nullptr || workspace_bytes < need))
        return fail(hipErrorInvalidValue,
                    "%s: workspace of %lld bytes given, %lld needed (ctattn_linear_bwd_workspace_bytes)", fn,
                    (long long)workspace_bytes, (long long)need);
    hipStream_t st = as_stream(stream);
    const bool v4 = linear_vec4(dtype, M, N, K, {x, w, dy, dx, dw});
    float *ws = static_cast<float *>(workspace);
    hipError_t e = hipSuccess;
    const int64_t split_bytes = linear_split_bytes(dtype, M, N, K);
    if (dw && lin_policy(dtype)) {
        ctattn::LinGemm g = lin_dw(dtype, x, dy, dw, M, N, K);
        g.db[0] = db;  // the bias gradient (column sums of dy) from the same launch
        if (ctattn::lin_gemm_supported(g)) {
            e = ctattn::launch_lin_gemm(g, workspace, split_bytes, st);
            if (e != hipSuccess) return finish(fn, e, st);
            dw = nullptr;
            db = nullptr;
        }
    }
    if (dw) {
        // dw[n][k] += sum_m dy[m][n] x[m][k]: M' = N, N' = K, K' = M.  A(m'=n, k'=m) = dy stored
        // [k'][m']; B(k'=m, n'=k) = x stored [k'][n'].
        const int splits = choose_splits(dtype, N, K, M, 1);
        GemmParams p = make_params(N, K, M, 1, splits, linear_view(nullptr, K), ws);
        p.batch[0].nseg = 1;
        p.batch[0].a[0] = linear_view(dy, N);
        p.batch[0].b[0] = linear_view(x, K);
        p.batch[0].out = dw;
        p.batch[0].bias = nullptr;
        e = ctattn::launch_proj_gemm(dtype, p, 1, false, false, v4, st);
        if (e != hipSuccess) return finish(fn, e, st);
    }
    if (db) {
        void *cws = static_cast<char *>(workspace) + split_bytes;
        e = ctattn::launch_colsum_add(dtype, linear_view(dy, N), int(M), int(N), db, cws, st);
        if (e != hipSuccess) return finish(fn, e, st);
    }
    if (dx && lin_policy(dtype)) {
        const ctattn::LinGemm g = lin_dx(dtype, dy, w, dx, M, N, K);
        if (ctattn::lin_gemm_supported(g)) return finish(fn, ctattn::launch_lin_gemm(g, nullptr, 0, st), st);
    }
    if (dx) {
        // dx[m][k] = sum_n dy[m][n] w[n][k]: A = dy [M][N] (K-contiguous), B = w stored [k'][n'].
        GemmParams p = make_params(M, K, N, 0, 1, linear_view(nullptr, K), nullptr);
        p.batch[0].nseg = 1;
        p.batch[0].a[0] = linear_view(dy, N);
        p.batch[0].b[0] = linear_view(w, K);
        p.batch[0].out = dx;
        p.batch[0].bias = nullptr;
        e = ctattn::launch_proj_gemm(dtype, p, 1, true, false, v4, st);
    }
    return finish(fn, e, st);
}

int ctattn_linear_act_fwd(int dtype, int act, const void *x, const void *w, const void *b, void *pre, void *y,
                          int64_t M, int64_t N, int64_t K, void *stream) {
    const char *fn = "ctattn_linear_act_fwd";
    if (int rc = validate_linear(fn, dtype, M, N, K)) return rc;
    if (act < CTATTN_ACT_RELU || act > CTATTN_ACT_TANH) return fail(hipErrorInvalidValue, "%s: unknown activation %d", fn, act);
    if (M == 0) return ok();
    if (!x || !w || !pre || !y) return fail(hipErrorInvalidValue, "%s: null x/w/pre/y pointer", fn);
    if (lin_policy(dtype)) {
        ctattn::LinGemm g = lin_fwd(dtype, x, w, b, pre, M, N, K);
        g.act_mode = 1;
        g.act_kind = act;
        g.aux[0] = y;
        if (ctattn::lin_gemm_supported(g))
            return finish(fn, ctattn::launch_lin_gemm(g, nullptr, 0, as_stream(stream)), as_stream(stream));
    }
    if (int rc = ctattn_linear_fwd(dtype, x, w, b, pre, M, N, K, stream)) return rc;
    return ctattn_activation_fwd(dtype, act, pre, y, M * N, stream);
}

int ctattn_linear_act_bwd(int dtype, int act, const void *x, const void *w, const void *dy, const void *pre,
                          void *dpre, void *dw, void *db, void *workspace, int64_t workspace_bytes, int64_t M,
                          int64_t N, int64_t K, void *stream) {
    const char *fn = "ctattn_linear_act_bwd";
    if (int rc = validate_linear(fn, dtype, M, N, K)) return rc;
    if (act < CTATTN_ACT_RELU || act > CTATTN_ACT_TANH) return fail(hipErrorInvalidValue, "%s: unknown activation %d", fn, act);
    if (M == 0) return ok();
    if (!dy || !w || !pre || !dpre) return fail(hipErrorInvalidValue, "%s: null dy/w/pre/dpre pointer", fn);
    if (dw || db) {
        if (int rc = ctattn_linear_bwd(dtype, x, w, dy, nullptr, dw, db, workspace, workspace_bytes, M, N, K, stream))
            return rc;
    }
    if (lin_policy(dtype)) {
        ctattn::LinGemm g = lin_dx(dtype, dy, w, dpre, M, N, K);
        g.act_mode = 2;
        g.act_kind = act;
        g.aux[0] = const_cast<void *>(pre);
        if (ctattn::lin_gemm_supported(g))
            return finish(fn, ctattn::launch_lin_gemm(g, nullptr, 0, as_stream(stream)), as_stream(stream));
    }
    if (int rc = ctattn_linear_bwd(dtype, x, w, dy, dpre, nullptr, nullptr, workspace, workspace_bytes, M, N, K, stream))
        return rc;
    return ctattn_activation_bwd(dtype, act, pre, dpre, dpre, M * K, stream);
}

int ctattn_sgd_update(int dtype, void *params, const void *grads, double lr, int64_t n, void *stream) {
    const char *fn = "ctattn_sgd_update";
    if (!known_dtype(dtype))
        return fail(hipErrorInvalidValue, "%s: unknown dtype %d (0 = f32, 1 = bf16, 2 = f16, 3 = f64)", fn, dtype);
    if (n < 0) return fail(hipErrorInvalidValue, "%s: negative size %lld", fn, (long long)n);
    if (n == 0) return ok();
    if (!params || !grads) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    if (double(n) > 2147483647.0 * 256.0) return fail(hipErrorInvalidValue, "%s: n too large", fn);
    hipStream_t st = as_stream(stream);
    return finish(fn, ctattn::launch_sgd(dtype, params, grads, lr, n, st), st);
}

}  // extern "C"
