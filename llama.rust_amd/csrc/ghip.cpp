// ghip.cpp -- host side of the gfx950 backend: code-object loading, operand
// validation, workspace management and kernel dispatch behind include/ghip.h.
#include "../../include/ghip.h"
#include "ghip_internal.h"

#include <hip/hip_runtime.h>

#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <strings.h>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

const char *const kModules[] = {"ghip_quant.hsaco", "ghip_gemv.hsaco", "ghip_wquant.hsaco", "ghip_gemm.hsaco", "ghip_fa.hsaco", "ghip_moe.hsaco", "ghip_skinny.hsaco", "ghip_iq.hsaco", "ghip_dense.hsaco"};

struct TypeInfo {
    int blck;
    int bytes;
};

TypeInfo type_info(int t) {
    switch (t) {
    case GHIP_TYPE_F32: return {1, 4};
    case GHIP_TYPE_F16: return {1, 2};
    case GHIP_TYPE_BF16: return {1, 2};
    case GHIP_TYPE_IQ2_XXS: return {256, 66};
    case GHIP_TYPE_IQ2_XS: return {256, 74};
    case GHIP_TYPE_IQ2_S: return {256, 82};
    case GHIP_TYPE_IQ3_XXS: return {256, 98};
    case GHIP_TYPE_IQ3_S: return {256, 110};
    case GHIP_TYPE_IQ1_S: return {256, 50};
    case GHIP_TYPE_IQ1_M: return {256, 56};
    case GHIP_TYPE_Q4_0: return {32, 18};
    case GHIP_TYPE_Q4_1: return {32, 20};
    case GHIP_TYPE_Q2_K: return {256, 84};
    case GHIP_TYPE_Q3_K: return {256, 110};
    case GHIP_TYPE_Q5_0: return {32, 22};
    case GHIP_TYPE_Q5_1: return {32, 24};
    case GHIP_TYPE_Q8_1: return {32, 36};
    case GHIP_TYPE_Q8_0: return {32, 34};
    case GHIP_TYPE_Q4_K: return {256, 144};
    case GHIP_TYPE_Q5_K: return {256, 176};
    case GHIP_TYPE_Q6_K: return {256, 210};
    case GHIP_TYPE_Q8_K: return {256, 292};
    case GHIP_TYPE_I32: return {1, 4};
    case GHIP_TYPE_MXFP4: return {32, 17};
    case GHIP_TYPE_IQ4_NL: return {32, 18};
    case GHIP_TYPE_IQ4_XS: return {256, 136};
    case GHIP_TYPE_NVFP4: return {64, 36};
    case GHIP_TYPE_Q1_0: return {128, 18};
    case GHIP_TYPE_Q2_0: return {64, 18};
    default: return {0, 0};
    }
}

std::string library_dir() {
    Dl_info info;
    if (dladdr((void *)&library_dir, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        const size_t s = p.rfind('/');
        if (s != std::string::npos) return p.substr(0, s);
    }
    return ".";
}

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

}  // namespace

struct ghip_context {
    int device = 0;
    std::vector<hipModule_t> modules;
    std::unordered_map<std::string, hipFunction_t> fns;
    std::string err;
    // Workspace (quantized activations, GEMM layouts, split partials, routing
    // tables).  Three sources, first match wins:
    //  - call_ws: the fixed scratch of a no-allocation entry point, for one call;
    //  - user_ws: caller memory given with ghip_set_workspace (never grown);
    //  - ws: owned by the library, grown on demand outside stream capture.
    void *ws = nullptr;
    size_t ws_size = 0;
    std::vector<void *> retired;  // outgrown owned workspaces: in-flight work or captured graphs may still read them
    void *user_ws = nullptr;
    size_t user_ws_size = 0;
    void *call_ws = nullptr;
    //  - hold: bytes at the start of the workspace that a ghip_graph_compute
    //    call keeps for its pre-quantized activations; the ops it runs get the
    //    workspace after them
    size_t hold = 0;
    size_t call_ws_size = 0;
    // the stream of the previous call: a call on another stream first waits
    // for it, so the two never share the workspace concurrently
    hipStream_t last_stream = nullptr;
    bool have_last = false;
    hipEvent_t order_ev = nullptr;
    std::mutex mu;
    // Device copies of registered weights in the layouts the kernels read
    // (ghip_weight_register), keyed by where and what the weight is.
    struct WeightKey {
        const void *data;
        int type;
        int64_t ne0, ne1, ne2;
        uint64_t nb1, nb2;
        bool operator==(const WeightKey &o) const {
            return data == o.data && type == o.type && ne0 == o.ne0 && ne1 == o.ne1 && ne2 == o.ne2 &&
                   nb1 == o.nb1 && nb2 == o.nb2;
        }
    };
    static WeightKey key_of(const ghip_tensor *w) {
        return {w->data, w->type, w->ne[0], w->ne[1], w->ne[2], w->nb[1], w->ne[2] > 1 ? w->nb[2] : 0};
    }
    struct WeightCopy {
        void *p;
        size_t bytes;
    };
    struct WeightKeyHash {
        size_t operator()(const WeightKey &k) const {
            size_t h = std::hash<const void *>()(k.data);
            h = h * 31 + (size_t)k.type;
            h = h * 31 + (size_t)k.ne0;
            h = h * 31 + (size_t)k.ne1;
            h = h * 31 + (size_t)k.ne2;
            return h * 31 + (size_t)k.nb1;
        }
    };
    std::unordered_map<WeightKey, WeightCopy, WeightKeyHash> wcache;
    // pinned host staging for ghip_gguf_upload: two buffers, each reused
    // once the copy engine has drained it (its event)
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t stage_ev[2] = {nullptr, nullptr};
    size_t wcache_bytes = 0;   // bytes held by wcache
    size_t wcache_built = 0;   // copies materialized so far (hits do not count)

    // Store check (GHIP_CHECK_STORES=1, and every dry-run context): before a
    // launch, the byte windows its kernel stores to -- worked out from the
    // launch's own arguments (expect) -- must lie inside the buffers the op
    // writes: its dst / sub-sum / activation outputs and the workspace it took
    // (allow).  A dry-run context (ghip_init_dry_run) has no device: ops plan,
    // take a workspace address range and check every launch without running it.
    bool check_stores = false;
    bool dry_run = false;
    struct Span {
        uintptr_t lo, hi;
        const char *what;
    };
    std::vector<Span> allowed, pending;
    void allow(const void *p, size_t n, const char *what) {
        if (check_stores && p && n) allowed.push_back({(uintptr_t)p, (uintptr_t)p + n, what});
    }
    void expect(const void *p, size_t n, const char *what) {
        if (check_stores && n) pending.push_back({(uintptr_t)p, (uintptr_t)p + n, what});
    }
    // the device current for an op (nothing to do in a dry run)
    bool set_device() { return dry_run || hipSetDevice(device) == hipSuccess; }

    ghip_status fail(ghip_status st, const char *fmt, ...) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        err = buf;
        return st;
    }

    hipFunction_t fn(const std::string &name) {
        auto it = fns.find(name);
        if (it != fns.end()) return it->second;
        for (hipModule_t m : modules) {
            hipFunction_t f = nullptr;
            if (hipModuleGetFunction(&f, m, name.c_str()) == hipSuccess && f) {
                fns[name] = f;
                return f;
            }
            (void)hipGetLastError();  // a miss in this module must not stay the thread's last error
        }
        return nullptr;
    }

    static bool capturing(hipStream_t s) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        return cs != hipStreamCaptureStatusNone;
    }

    // Called at the start of every op on stream s (device current, lock held).
    ghip_status begin(hipStream_t s) {
        allowed.clear();
        pending.clear();
        if (dry_run) return GHIP_STATUS_SUCCESS;
        if (have_last && last_stream != s && !capturing(s) && !capturing(last_stream)) {
            if (hipEventRecord(order_ev, last_stream) != hipSuccess || hipStreamWaitEvent(s, order_ev, 0) != hipSuccess) {
                (void)hipGetLastError();
                return fail(GHIP_STATUS_BACKEND_ERROR, "cannot order stream %p after %p", (void *)s, (void *)last_stream);
            }
        }
        last_stream = s;
        have_last = true;
        return GHIP_STATUS_SUCCESS;
    }

    ghip_status workspace(size_t bytes, hipStream_t s, void **out) {
        ghip_status st = workspace_get(bytes, s, out);
        if (st == GHIP_STATUS_SUCCESS) allow(*out, bytes, "workspace");
        return st;
    }
    ghip_status workspace_get(size_t bytes, hipStream_t s, void **out) {
        ghip_status st = workspace_base(bytes + hold, s, out);
        if (st == GHIP_STATUS_SUCCESS) *out = (uint8_t *)*out + hold;
        return st;
    }
    ghip_status workspace_base(size_t bytes, hipStream_t s, void **out) {
        if (dry_run && !call_ws && !user_ws) {
            // an address range no allocation uses: the launches are checked, never run
            *out = (void *)(uintptr_t)(1ull << 46);
            return GHIP_STATUS_SUCCESS;
        }
        if (call_ws) {
            if (bytes > call_ws_size)
                return fail(GHIP_STATUS_ALLOC_FAILED, "this call needs %zu bytes of scratch; the fixed scratch holds %zu",
                            bytes, call_ws_size);
            *out = call_ws;
            return GHIP_STATUS_SUCCESS;
        }
        if (user_ws) {
            if (bytes > user_ws_size)
                return fail(GHIP_STATUS_ALLOC_FAILED,
                            "this call needs %zu bytes of workspace; ghip_set_workspace gave %zu", bytes, user_ws_size);
            *out = user_ws;
            return GHIP_STATUS_SUCCESS;
        }
        if (bytes > ws_size) {
            if (capturing(s))
                return fail(GHIP_STATUS_ALLOC_FAILED,
                            "the workspace must grow to %zu bytes while the stream is being captured: run the same "
                            "call once before capturing, or give a workspace with ghip_set_workspace",
                            bytes);
            size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
            want = std::max(want, ws_size + ws_size / 2);
            void *p = nullptr;
            if (hipMalloc(&p, want) != hipSuccess) {
                (void)hipGetLastError();
                return fail(GHIP_STATUS_OUT_OF_MEMORY, "workspace hipMalloc(%zu) failed", want);
            }
            // the old buffer is kept until ghip_free: queued kernels and
            // captured graphs may still point at it
            if (ws) retired.push_back(ws);
            ws = p;
            ws_size = want;
        }
        *out = ws;
        return GHIP_STATUS_SUCCESS;
    }

    template <typename... Args>
    ghip_status launch(const std::string &name, dim3 grid, dim3 block, size_t shmem, hipStream_t s,
                       Args... args) {
        if (check_stores) {
            for (const Span &w : pending) {
                bool inside = false;
                for (const Span &a : allowed) inside = inside || (w.lo >= a.lo && w.hi <= a.hi);
                if (!inside) {
                    pending.clear();
                    return fail(GHIP_STATUS_BACKEND_ERROR,
                                "store check: %s of %s would store %zu bytes at %p, outside every buffer of this op",
                                w.what, name.c_str(), (size_t)(w.hi - w.lo), (void *)w.lo);
                }
            }
            pending.clear();
        }
        if (dry_run) return GHIP_STATUS_SUCCESS;
        hipFunction_t f = fn(name);
        if (!f) return fail(GHIP_STATUS_BACKEND_ERROR, "kernel %s not found in the code objects", name.c_str());
        void *ptrs[] = {(void *)&args...};
        const hipError_t e =
            hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, (unsigned)shmem, s, ptrs, nullptr);
        if (e != hipSuccess)
            return fail(GHIP_STATUS_BACKEND_ERROR, "launch of %s failed: %s", name.c_str(), hipGetErrorString(e));
        return GHIP_STATUS_SUCCESS;
    }
};

namespace {

// ----------------------------------------------------------- MUL_MAT plans

struct MulMatPlan {
    int wtype;        // src0 type
    int64_t K, N, M;  // ne00, ne01, ne11
    int64_t w_row_bytes;
    int act_type;     // Q8_0 or Q8_K
    int64_t act_row_bytes;
    int64_t n_mat;    // leading activation rows quantized with quantize_mat_q8_K_4x8 values
    int64_t nb;       // blocks per weight row
    bool act_pre;     // src1 already holds the vec_dot_type blocks
};

// IQ1 / IQ2 / IQ3 codebook weights (ghip_iq.hip gemv_grid_impl), Q8_K activations
bool grid_type(int t) {
    return t == GHIP_TYPE_IQ2_XXS || t == GHIP_TYPE_IQ2_XS || t == GHIP_TYPE_IQ2_S || t == GHIP_TYPE_IQ3_XXS ||
           t == GHIP_TYPE_IQ3_S || t == GHIP_TYPE_IQ1_S || t == GHIP_TYPE_IQ1_M;
}
// F32 / F16 / BF16 weights (ghip_dense.hip)
bool dense_type(int t) { return t == GHIP_TYPE_F32 || t == GHIP_TYPE_F16 || t == GHIP_TYPE_BF16; }
bool plan_mul_mat(ghip_context *ctx, const ghip_tensor *a, const ghip_tensor *b, const ghip_tensor *d,
                  MulMatPlan &p, ghip_status &st) {
    st = GHIP_STATUS_BACKEND_ERROR;
    if (!a || !b) { st = ctx->fail(st, "mul_mat: null operand"); return false; }
    if (a->type != GHIP_TYPE_Q4_0 && a->type != GHIP_TYPE_Q5_0 && a->type != GHIP_TYPE_Q8_0 &&
        a->type != GHIP_TYPE_Q4_K && a->type != GHIP_TYPE_Q5_K && a->type != GHIP_TYPE_Q6_K &&
        a->type != GHIP_TYPE_Q4_1 && a->type != GHIP_TYPE_Q5_1 && a->type != GHIP_TYPE_Q2_K &&
        a->type != GHIP_TYPE_Q3_K && a->type != GHIP_TYPE_IQ4_NL && a->type != GHIP_TYPE_IQ4_XS &&
        a->type != GHIP_TYPE_NVFP4 && a->type != GHIP_TYPE_Q1_0 && a->type != GHIP_TYPE_Q2_0 &&
        a->type != GHIP_TYPE_F32 && a->type != GHIP_TYPE_F16 && a->type != GHIP_TYPE_BF16 && !grid_type(a->type)) {
        st = ctx->fail(st,
                       "mul_mat: src0 type %d not supported (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, "
                       "IQ4_NL, IQ4_XS, NVFP4, Q1_0, Q2_0, IQ1_S, IQ1_M, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, F32, F16, BF16)",
                       a->type);
        return false;
    }
    const TypeInfo ti = type_info(a->type);
    // vec_dot_type Q8_0 (vec_dot.rs:1727): Q4_0, Q5_0, Q8_0, NVFP4, IQ4_NL
    const bool q8_0_dot = a->type == GHIP_TYPE_Q4_0 || a->type == GHIP_TYPE_Q5_0 || a->type == GHIP_TYPE_Q8_0 ||
                          a->type == GHIP_TYPE_IQ4_NL || a->type == GHIP_TYPE_NVFP4 || a->type == GHIP_TYPE_Q1_0 ||
                          a->type == GHIP_TYPE_Q2_0;
    const bool q8_1_dot = a->type == GHIP_TYPE_Q4_1 || a->type == GHIP_TYPE_Q5_1;
    const bool dense = dense_type(a->type);
    // vec_dot_type (vec_dot.rs vec_dot_type); F32 / F16 / BF16 weights take the
    // f32 src1 and round it themselves (compute.rs:1700-1745)
    const int vdt = dense ? GHIP_TYPE_F32 : q8_0_dot ? GHIP_TYPE_Q8_0 : q8_1_dot ? GHIP_TYPE_Q8_1 : GHIP_TYPE_Q8_K;
    if (b->type != GHIP_TYPE_F32 && b->type != vdt) {
        st = ctx->fail(st, "mul_mat: src1 must be F32 or the vec_dot type of src0 (backend.rs:2057-2066)");
        return false;
    }
    if (a->ne[0] != b->ne[0]) { st = ctx->fail(st, "mul_mat: ne00 != ne10"); return false; }
    if (a->ne[0] % ti.blck) { st = ctx->fail(st, "mul_mat: ne00 %% block size != 0"); return false; }
    if (a->ne[0] <= 0) { st = ctx->fail(st, "mul_mat: ne00 must be positive"); return false; }
    if ((int64_t)a->nb[0] != ti.bytes) { st = ctx->fail(st, "mul_mat: permuted src0 (nb0 != type size)"); return false; }
    if ((int64_t)b->nb[0] != type_info(b->type).bytes) { st = ctx->fail(st, "mul_mat: permuted src1"); return false; }
    // batches: dst plane (i12, i13) = src0 plane (i12 / r2, i13 / r3) x src1
    // plane (i12, i13), r2 = ne12 / ne02, r3 = ne13 / ne03 (compute.rs:1440-1450);
    // mul_mat_impl runs the planes one by one
    if (a->ne[2] < 1 || a->ne[3] < 1 || b->ne[2] < 0 || b->ne[3] < 0 || b->ne[2] % a->ne[2] ||
        b->ne[3] % a->ne[3]) {
        st = ctx->fail(st, "mul_mat: src1 planes (ne12, ne13) must be multiples of src0's (ne02, ne03)");
        return false;
    }
    if (b->type == GHIP_TYPE_F32 && b->nb[1] % 4) { st = ctx->fail(st, "mul_mat: src1 row stride not a multiple of 4"); return false; }
    if (d) {
        if (d->type != GHIP_TYPE_F32 || d->nb[0] != 4 || d->ne[0] != a->ne[1] || d->ne[1] != b->ne[1] ||
            d->ne[2] != b->ne[2] || d->ne[3] != b->ne[3] || d->nb[1] % 4) {
            st = ctx->fail(st, "mul_mat: dst must be F32 [ne01, ne11, ne12, ne13] with nb0 == 4");
            return false;
        }
    }
    p.wtype = a->type;
    p.K = a->ne[0];
    p.N = a->ne[1];
    p.M = b->ne[1];
    p.nb = p.K / ti.blck;
    p.w_row_bytes = (int64_t)a->nb[1];
    if (p.w_row_bytes < p.nb * ti.bytes) { st = ctx->fail(st, "mul_mat: src0 nb1 too small"); return false; }
    if (dense) {
        p.act_type = GHIP_TYPE_F32;
        p.act_row_bytes = p.K * 4;
        p.n_mat = 0;
    } else if (q8_0_dot) {
        p.act_type = GHIP_TYPE_Q8_0;
        p.act_row_bytes = p.K / 32 * 34;
        p.n_mat = 0;
    } else if (q8_1_dot) {
        p.act_type = GHIP_TYPE_Q8_1;
        p.act_row_bytes = p.K / 32 * 36;
        p.n_mat = 0;
    } else {
        p.act_type = GHIP_TYPE_Q8_K;
        p.act_row_bytes = p.K / 256 * 292;
        // repacked Q4_K (ne01 % 8 == 0): quantize_mat_q8_K_4x8 for ne11 - ne11 % 4 rows
        p.n_mat = (a->type == GHIP_TYPE_Q4_K && p.N % 8 == 0) ? p.M - p.M % 4 : 0;
    }
    p.act_pre = b->type != GHIP_TYPE_F32;
    if (p.act_pre) p.act_row_bytes = (int64_t)b->nb[1];
    if (p.N > INT32_MAX || p.nb > INT32_MAX) { st = ctx->fail(st, "mul_mat: dimension too large"); return false; }
    if (p.M < 0 || p.N < 0) { st = ctx->fail(st, "mul_mat: negative dimension"); return false; }
    st = GHIP_STATUS_SUCCESS;
    return true;
}

ghip_status quantize_act(ghip_context *ctx, const MulMatPlan &p, const ghip_tensor *b, void *out, hipStream_t s) {
    const int64_t x_stride = (int64_t)b->nb[1] / 4;
    ctx->expect(out, (size_t)(p.M * p.act_row_bytes), "quantized activations");
    if (p.act_type == GHIP_TYPE_Q8_K) {
        const int64_t waves = p.M * (p.K / 256);
        const unsigned grid = (unsigned)((waves + 3) / 4);
        return ctx->launch("ghip_quantize_q8_K", dim3(grid), dim3(256), 0, s, (const float *)b->data, x_stride,
                           (int64_t)p.K, (int64_t)p.M, (uint8_t *)out, (int64_t)p.act_row_bytes, (int64_t)p.n_mat);
    }
    const int64_t blocks = p.M * (p.K / 32);
    const unsigned grid = (unsigned)((blocks * 8 + 255) / 256);
    return ctx->launch(p.act_type == GHIP_TYPE_Q8_1 ? "ghip_quantize_q8_1" : "ghip_quantize_q8_0", dim3(grid),
                       dim3(256), 0, s, (const float *)b->data, x_stride, (int64_t)p.K, (int64_t)p.M, (uint8_t *)out,
                       (int64_t)p.act_row_bytes);
}

const char *gemv_base(int wtype) {
    switch (wtype) {
    case GHIP_TYPE_Q4_K: return "ghip_gemv_q4_K";
    case GHIP_TYPE_Q5_K: return "ghip_gemv_q5_K";
    case GHIP_TYPE_Q6_K: return "ghip_gemv_q6_K";
    case GHIP_TYPE_Q5_0: return "ghip_gemv_q5_0";
    case GHIP_TYPE_Q8_0: return "ghip_gemv_q8_0";
    case GHIP_TYPE_Q4_1: return "ghip_gemv_q4_1";
    case GHIP_TYPE_Q2_K: return "ghip_gemv_q2_K";
    case GHIP_TYPE_Q3_K: return "ghip_gemv_q3_K";
    case GHIP_TYPE_Q5_1: return "ghip_gemv_q5_1";
    case GHIP_TYPE_IQ4_NL: return "ghip_gemv_iq4_nl";
    case GHIP_TYPE_IQ4_XS: return "ghip_gemv_iq4_xs";
    case GHIP_TYPE_NVFP4: return "ghip_gemv_nvfp4";
    case GHIP_TYPE_Q1_0: return "ghip_gemv_q1_0";
    case GHIP_TYPE_Q2_0: return "ghip_gemv_q2_0";
    case GHIP_TYPE_IQ2_XXS: return "ghip_gemv_iq2_xxs";
    case GHIP_TYPE_IQ2_XS: return "ghip_gemv_iq2_xs";
    case GHIP_TYPE_IQ2_S: return "ghip_gemv_iq2_s";
    case GHIP_TYPE_IQ3_XXS: return "ghip_gemv_iq3_xxs";
    case GHIP_TYPE_IQ3_S: return "ghip_gemv_iq3_s";
    case GHIP_TYPE_IQ1_S: return "ghip_gemv_iq1_s";
    case GHIP_TYPE_IQ1_M: return "ghip_gemv_iq1_m";
    default: return "ghip_gemv_q4_0";
    }
}

// Q2_K / Q3_K: the VALU decode kernel in launches of at most 4 columns
bool k23_type(int wtype) { return wtype == GHIP_TYPE_Q2_K || wtype == GHIP_TYPE_Q3_K; }

// 32-element blocks with Q8_0 activations: one lane per pair of blocks
bool gemv_pair(int wtype) {
    return wtype == GHIP_TYPE_Q4_0 || wtype == GHIP_TYPE_Q5_0 || wtype == GHIP_TYPE_Q8_0;
}
// table-lookup 4-bit and 1-/2-bit code types (ghip_iq.hip): one decode lane per 32 elements
bool lut_type(int wtype) {
    return wtype == GHIP_TYPE_IQ4_NL || wtype == GHIP_TYPE_IQ4_XS || wtype == GHIP_TYPE_NVFP4 ||
           wtype == GHIP_TYPE_Q1_0 || wtype == GHIP_TYPE_Q2_0 || grid_type(wtype);
}
// weights the int8-MFMA GEMM ghip_gemm_q8 takes as int8 codes with one scale
// per 32 elements (NVFP4's scales are per 16: its prefill runs the decode
// kernel in groups of 8 columns)
bool gemm_q8_family(int wtype) {
    return gemv_pair(wtype) || wtype == GHIP_TYPE_IQ4_NL || wtype == GHIP_TYPE_IQ4_XS || wtype == GHIP_TYPE_Q1_0 ||
           wtype == GHIP_TYPE_Q2_0;
}
// int32 sub-sums per weight block (ghip_mul_mat_subsums layout)
// bytes a kernel covers storing m rows of n elements at stride ldd
size_t win2d(int64_t m, int64_t ldd, int64_t n, size_t e = 4) {
    return m > 0 && n > 0 ? ((size_t)(m - 1) * (size_t)ldd + (size_t)n) * e : 0;
}
int64_t subsums_per_block(int wtype) {
    if (wtype == GHIP_TYPE_Q4_K || wtype == GHIP_TYPE_Q5_K || wtype == GHIP_TYPE_Q2_K) return 2;
    return wtype == GHIP_TYPE_NVFP4 || wtype == GHIP_TYPE_Q1_0 ? 4 : wtype == GHIP_TYPE_Q2_0 ? 2 : 1;
}
// int32 sub-sums of m activation rows
size_t sub_bytes(const MulMatPlan &p, int64_t m) {
    return (size_t)m * (size_t)p.N * (size_t)p.nb * (size_t)subsums_per_block(p.wtype) * 4;
}

// The whole-row decode kernels with the activation image in LDS: Q4_K and
// Q5_K always; Q6_K for a single activation row (its 14336-wide rows make the
// per-workgroup quantization of several columns cost more than it saves).
bool gemv_v2(const MulMatPlan &p) {
    return p.wtype == GHIP_TYPE_Q4_K || p.wtype == GHIP_TYPE_Q5_K || (p.wtype == GHIP_TYPE_Q6_K && p.M == 1);
}

// Row groups of the whole-row decode kernels (RB rows per register group, NG
// groups per row team, streamed two deep).  Batch 1 streams one-row groups
// deeper on large matrices: Q4_K 4096 -> 14336 9.6 -> 9.2 us, Q6_K 14336 ->
// 4096 16.0 -> 14.8 us; smaller matrices keep 2 x 2 (4096 -> 4096: 4.5 us
// against 5.2 with 1 x 4).
// Q4_K at one or two activation rows with K in one wavefront: one-row groups, teams
// and rows per team chosen for about 256 workgroups (one per CU), ns groups
// loaded before the activation is quantized.  Measured (graph-timed, rotating
// weights): 4096 -> 14336 9.0 -> 8.2 us (1 x 7, 3 slots), 4096 -> 4096
// 4.6 -> 4.5 us, 4096 -> 1024 4.2 -> 3.6 us (1 x 2, 4 teams); at two rows
// 4096 -> 14336 12.0 -> 10.2 us, 4096 -> 4096 6.3 -> 6.1 us.
void gemv_q4k_one_row(int64_t rows, int &teams, int &ng, int &ns) {
    teams = rows >= 4096 ? 8 : 4;
    const int64_t per_team = (rows + 256 * teams - 1) / (256 * teams);
    if (per_team <= 2) ng = 2, ns = 2;
    else if (per_team <= 4) ng = 4, ns = 3;
    else if (per_team <= 7) ng = 7, ns = 3;
    else ng = 8, ns = 3;
}

void gemv_groups(int wtype, int64_t M, int64_t N, int &rb, int &ng) {
    rb = 2;
    ng = 2;
    if (M != 1) return;
    if (wtype == GHIP_TYPE_Q6_K) rb = 1, ng = 8;
    else if (wtype == GHIP_TYPE_Q4_K && N >= 8192) rb = 1, ng = 4;
}

// Q4_K at 2..15 activation rows on the int8 matrix cores (ghip_skinny.hip):
// RT row tiles of 16 rows x KS K-slices per 8-wavefront workgroup, tokens
// padded to NC in {2, 4, 8, 16}.
// From 4 rows (at 2 and 3 the VALU kernels are as fast).  The activation
// rows are quantized once by ghip_quantize_q8_K and copied into each
// workgroup's LDS: quantizing them in every workgroup cost 5.6 us of 21.2 at
// 8 rows on 4096 -> 14336 (15.6 us with the rows quantized once).
// At 3-4 rows on matrices under 8192 rows (K in one wavefront) the VALU
// kernel with one-row groups is faster: 4096 -> 4096 at 4 rows 10.9 -> 8.6 us.
bool valu_q4k_small(const MulMatPlan &p) {
    return p.wtype == GHIP_TYPE_Q4_K && p.M <= 4 && p.N < 8192 && p.nb <= 16;
}
void skinny_shape(int64_t M, int &NC, int &RT, int &KS);
size_t skinny_lds(int NC, int64_t K, int64_t nb);
// (9-15 rows of a long K, e.g. 14336 at 16 columns, do not fit the LDS
// image: they take the whole-row kernels in groups of 8 columns)
bool use_skinny(const MulMatPlan &p) {
    if (!(p.wtype == GHIP_TYPE_Q4_K && p.M >= env_int("GHIP_MMA_MIN_ROWS", 4) && p.M < 16 &&
          env_int("GHIP_MMA", 1) != 0 && !valu_q4k_small(p)))
        return false;
    int NC, RT, KS;
    skinny_shape(p.M, NC, RT, KS);
    return skinny_lds(NC, p.K, p.nb) <= 160 * 1024;
}
// The K split sets the fp32 summation order, so it is fixed (2 row tiles x
// 4 K-slices) for every matrix size: a matrix alone and in a grouped launch
// give the same bits.  GHIP_MMA_RT=1|4 overrides it (single-op calls only).
// Measured at 8 rows (pre-quantized): 4096 -> 14336 15.6 us (1 x 8: 20.0),
// 4096 -> 4096 9.1 us (1 x 8: 7.4).
void skinny_shape(int64_t M, int &NC, int &RT, int &KS) {
    NC = M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16;
    RT = env_int("GHIP_MMA_RT", 2);
    if (RT != 1 && RT != 2 && RT != 4) RT = 2;
    KS = 8 / RT;
}
size_t skinny_lds(int NC, int64_t K, int64_t nb) {
    return (size_t)NC * K + (size_t)NC * nb * 4 + (size_t)NC * nb * 16 * 4 + (size_t)8 * 16 * 16 * 4;
}
ghip_status run_skinny(ghip_context *ctx, const MulMatPlan &p, const void *w, const uint8_t *act, int64_t act_rb,
                       bool fused, float *dst, int64_t ldd, int32_t *sub, hipStream_t s) {
    int NC, RT, KS;
    skinny_shape(p.M, NC, RT, KS);
    const size_t shmem = skinny_lds(NC, p.K, p.nb);
    if (shmem > 160 * 1024) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: decode LDS image too large");
    const std::string name = std::string("ghip_mma_q4_K") + (fused ? "_f" : "") + (sub ? "_sub" : "") + "_c" +
                             std::to_string(NC) + "_r" + std::to_string(RT) + "k" + std::to_string(KS);
    const unsigned grid = (unsigned)((p.N + 16 * RT - 1) / (16 * RT));
    const int n_mat = (int)std::max<int64_t>(0, std::min<int64_t>(p.M, p.n_mat));
    ctx->expect(dst, win2d(p.M, ldd, p.N), "dst");
    if (sub) ctx->expect(sub, sub_bytes(p, p.M), "sub-sums");
    return ctx->launch(name, dim3(grid), dim3(512), shmem, s, (const uint8_t *)w, (int64_t)p.w_row_bytes, (int)p.N,
                       (int)p.nb, act, act_rb, (int)p.M, dst, ldd, sub, n_mat);
}

// Split-K decode (ghip_skinny.hip ghip_sk_*): Q4_K and Q6_K at 4..8 f32
// activation rows.  K-slices of S super-blocks (S from K alone: 4 up to 24
// super-blocks, else 8) x 64-row tiles; each workgroup quantizes its slice of
// the activations once (no quantize launch) and walks a set of tiles with
// the next step's weights in flight; ghip_sk_reduce adds the slices'
// partials in order.  GHIP_SK_WGS sets the workgroups aimed for (768: three
// per CU).
constexpr int kSkRows = 64;
int sk_sb(int64_t nb) { return nb <= 24 ? 4 : 8; }
int64_t sk_slices(int64_t nb) { return (nb + sk_sb(nb) - 1) / sk_sb(nb); }
int64_t sk_tiles(int64_t N) { return (N + kSkRows - 1) / kSkRows; }
// Q4_K below GHIP_SK_MIN_ROWS (8192) weight rows keeps the whole-K kernel
// (ghip_mma_q4_K_*) after one quantize launch: there the split kernel plus its
// reduction measured slower (q/k/v 14.3 -> 17.6 us, o 14.4 -> 14.6 us;
// gate/up 33.9 -> 29.1 us and Q6_K down 35.5 -> 28.1 us, both with the
// reduction).  sk_rows_ok is the row test alone (graph grouping keeps it
// equal within a group).
bool sk_rows_ok(int wtype, int64_t N) { return wtype == GHIP_TYPE_Q6_K || N >= env_int("GHIP_SK_MIN_ROWS", 8192); }
// Whole-K decode (ghip_skinny.hip ghip_sq_*): Q4_K and Q6_K at 4..8
// activation rows from ready Q8_K rows (one ghip_quantize_q8_K launch, shared
// by a group's members, or a Q8_K src1 as it is).  Workgroups of
// W = ceil(nb / SW) wavefronts, wavefront w on super-blocks [w SW, w SW + SW),
// T tiles of 16 weight rows each; the K-slices' partials are added inside the
// workgroup.  SW: 2 up to 32 super-blocks, 4 up to 56 (the LDS images of the
// W wavefronts, sq_img_bytes each, within 160 KB); longer rows take split K.
int sq_sw(int64_t nb) { return nb <= 32 ? 2 : nb <= 56 ? 4 : 0; }
size_t sq_img_bytes(int sw) {
    return (size_t)8 * (sw * 256 + 16) + (size_t)8 * sw * 4 + (size_t)8 * (sw * 16 + 4) * 4 + (size_t)sw * 256;
}
bool use_sq(const MulMatPlan &p) {
    return env_int("GHIP_SQ", 1) != 0 && (p.wtype == GHIP_TYPE_Q4_K || p.wtype == GHIP_TYPE_Q6_K) &&
           p.M >= env_int("GHIP_SQ_MIN_COLS", 4) && p.M <= 8 && sq_sw(p.nb) > 0;
}
// Q4_K takes split K from 5 rows: at 4 rows the matrix-core decode kernel is
// faster (4096 -> 14336: 17.2 us split K, 15.6 us).
// The whole-row decode kernels keep the activation rows' Q8_K image in LDS
// (codes, scales and 16-element sums of up to 8 rows); past 160 KB (8 rows of
// K > 15.5 K) only split K can take the matrix, whatever its row count.
bool decode_image_fits(const MulMatPlan &p) {
    const int64_t NC = p.M <= 1 ? 1 : p.M <= 2 ? 2 : p.M <= 4 ? 4 : 8;
    return NC * p.K + NC * p.nb * 4 + NC * p.nb * 16 * 4 + 8 * 16 * 16 * 4 <= 160 * 1024;
}
bool use_sk(const MulMatPlan &p) {
    if (use_sq(p)) return false;
    if (p.act_pre || env_int("GHIP_SK", 1) == 0 || p.M < env_int("GHIP_MMA_MIN_ROWS", 4)) return false;
    if (p.wtype == GHIP_TYPE_Q4_K && p.M < env_int("GHIP_SK_Q4K_MIN_COLS", 5)) return false;
    return (p.wtype == GHIP_TYPE_Q4_K || p.wtype == GHIP_TYPE_Q6_K) && p.M <= 8 &&
           (sk_rows_ok(p.wtype, p.N) || !decode_image_fits(p));
}
size_t sk_part_bytes(const MulMatPlan &p) {
    const int64_t ns = sk_slices(p.nb);
    return ns > 1 ? (((size_t)ns * (size_t)p.M * (size_t)p.N * 4 + 255) & ~(size_t)255) : 0;
}
// Host mirror of SkMember / SkLaunch in ghip_skinny.hip.
struct SkMember {
    const uint8_t *W;
    float *dst;
    int64_t ldd;
    float *part;
    int rows;
    int tile0;
};
struct SkLaunch {
    SkMember m[4];
    int n, n_tiles, nks, tg;
};
// g: members' W, dst, ldd, rows and part filled in; launches the kernel and
// (more than one K-slice) the in-order reduction
ghip_status launch_sk(ghip_context *ctx, const MulMatPlan &p, SkLaunch &g, const ghip_tensor *x, int32_t *sub,
                      hipStream_t s) {
    const int64_t ns = sk_slices(p.nb);
    int64_t tiles = 0, rows = 0;
    SkLaunch r = g;  // the reduction's view: tile0 = first row
    for (int i = 0; i < 4; i++) {
        if (i >= g.n) g.m[i] = g.m[0], r.m[i] = r.m[0];
        g.m[i].tile0 = (int)tiles;
        r.m[i].tile0 = (int)rows;
        if (i < g.n) {
            tiles += sk_tiles(g.m[i].rows);
            rows += g.m[i].rows;
        }
    }
    if (rows * p.M > INT32_MAX || tiles * ns > INT32_MAX)
        return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: matrix too large for the split-K decode kernel");
    const int64_t want = std::max(1, env_int("GHIP_SK_WGS", 768));
    g.n_tiles = (int)tiles;
    g.nks = (int)ns;
    g.tg = (int)std::max<int64_t>(1, std::min<int64_t>(tiles, (want + ns - 1) / ns));
    r.nks = g.nks;
    const int n_mat = (int)std::max<int64_t>(0, std::min<int64_t>(p.M, p.n_mat));
    for (int i = 0; i < g.n; i++) {
        if (ns > 1) ctx->expect(g.m[i].part, (size_t)ns * (size_t)p.M * (size_t)g.m[i].rows * 4, "split-K partials");
        else ctx->expect(g.m[i].dst, win2d(p.M, g.m[i].ldd, g.m[i].rows), "dst");
    }
    if (sub) ctx->expect(sub, sub_bytes(p, p.M), "sub-sums");
    const std::string name = std::string("ghip_sk_") + (p.wtype == GHIP_TYPE_Q4_K ? "q4_K" : "q6_K") +
                             (sub ? "_sub" : "") + "_s" + std::to_string(sk_sb(p.nb));
    ghip_status st = ctx->launch(name, dim3((unsigned)(ns * g.tg)), dim3(256), 0, s, g, (int64_t)p.w_row_bytes,
                                 (int)p.nb, (const float *)x->data, (int64_t)x->nb[1] / 4, (int)p.M, n_mat, sub);
    if (st != GHIP_STATUS_SUCCESS || ns == 1) return st;
    const int64_t total = rows * p.M;
    for (int i = 0; i < g.n; i++) ctx->expect(r.m[i].dst, win2d(p.M, r.m[i].ldd, r.m[i].rows), "dst");
    return ctx->launch("ghip_sk_reduce", dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, r, (int)p.M, total);
}
// g: members' W, dst, ldd and rows filled in; act: the Q8_K rows (row stride act_rb)
ghip_status launch_sq(ghip_context *ctx, const MulMatPlan &p, SkLaunch &g, const uint8_t *act, int64_t act_rb,
                      int32_t *sub, hipStream_t s) {
    const int sw = sq_sw(p.nb);
    const int W = (int)((p.nb + sw - 1) / sw);
    int64_t tiles = 0;
    for (int i = 0; i < 4; i++) {
        if (i >= g.n) g.m[i] = g.m[0];
        g.m[i].tile0 = (int)tiles;
        g.m[i].part = nullptr;
        if (i < g.n) tiles += (g.m[i].rows + 15) / 16;
    }
    if (tiles * 16 * p.M > INT32_MAX) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: matrix too large for the decode kernel");
    if (sw == 2 && env_int("GHIP_SQ_STREAM", 1) != 0) {
        // streaming form: T tiles per workgroup for about GHIP_SQ_WGS workgroups
        // (256: one per CU; on the Llama-3-8B decode layer at 8 rows 160 / 192 /
        // 256 / 320 / 384 measured 79.0 / 74.2 / 68.9 / 78.2 / 75.1 us), within
        // the LDS (image + T tiles of partials per wavefront)
        const int64_t want = std::max(1, env_int("GHIP_SQ_WGS", 256));
        const size_t img = sq_img_bytes(sw);
        int64_t T = env_int("GHIP_SQ_T", (int)((tiles + want - 1) / want));
        T = std::max<int64_t>(1, std::min<int64_t>(T, (int64_t)((160 * 1024 / W - img) / 512)));
        g.n_tiles = (int)tiles;
        g.nks = 1;
        g.tg = (int)T;
        for (int i = 0; i < g.n; i++) ctx->expect(g.m[i].dst, win2d(p.M, g.m[i].ldd, g.m[i].rows), "dst");
        if (sub) ctx->expect(sub, sub_bytes(p, p.M), "sub-sums");
        const std::string name = std::string("ghip_sqs_") + (p.wtype == GHIP_TYPE_Q4_K ? "q4_K" : "q6_K") +
                                 (sub ? "_sub" : "") + "_w2";
        return ctx->launch(name, dim3((unsigned)((tiles + T - 1) / T)), dim3(64 * W), W * (img + (size_t)T * 512), s, g,
                           (int)T, (int64_t)p.w_row_bytes, (int)p.nb, act, act_rb, (int)p.M, sub);
    }
    // two tiles per workgroup from 1024 tiles at SW = 2 (the T = 2 kernels there)
    int T = env_int("GHIP_SQ_T", sw == 2 && tiles >= 1024 ? 2 : 1);
    if (T != 1 && !(T == 2 && sw == 2)) T = 1;
    g.n_tiles = (int)tiles;
    g.nks = 1;
    g.tg = T;
    for (int i = 0; i < g.n; i++) ctx->expect(g.m[i].dst, win2d(p.M, g.m[i].ldd, g.m[i].rows), "dst");
    if (sub) ctx->expect(sub, sub_bytes(p, p.M), "sub-sums");
    const std::string name = std::string("ghip_sq_") + (p.wtype == GHIP_TYPE_Q4_K ? "q4_K" : "q6_K") +
                             (sub ? "_sub" : "") + "_w" + std::to_string(sw) + "_t" + std::to_string(T);
    return ctx->launch(name, dim3((unsigned)((tiles + T - 1) / T)), dim3(64 * W), W * sq_img_bytes(sw), s, g,
                       (int64_t)p.w_row_bytes, (int)p.nb, act, act_rb, (int)p.M, sub);
}
ghip_status run_sk(ghip_context *ctx, const MulMatPlan &p, const void *w, const ghip_tensor *x, float *dst,
                   int64_t ldd, int32_t *sub, void *part, hipStream_t s) {
    SkLaunch g{};
    g.n = 1;
    g.m[0].W = (const uint8_t *)w;
    g.m[0].dst = dst;
    g.m[0].ldd = ldd;
    g.m[0].part = (float *)part;
    g.m[0].rows = (int)p.N;
    return launch_sk(ctx, p, g, x, sub, s);
}

// Decode path: activation columns in groups of at most 8.  Q4_K reads the f32
// activations and quantizes them inside the kernel when fused is set.
ghip_status run_gemv(ghip_context *ctx, const MulMatPlan &p, const void *w, const uint8_t *act, int64_t act_rb,
                     bool fused, float *dst, int64_t ldd, int32_t *sub, hipStream_t s) {
    if (use_skinny(p)) return run_skinny(ctx, p, w, act, act_rb, fused, dst, ldd, sub, s);
    int waves_k;
    if (gemv_pair(p.wtype))
        waves_k = (int)(((p.nb + 1) / 2 + 63) / 64);
    else if (p.wtype == GHIP_TYPE_Q4_1 || p.wtype == GHIP_TYPE_Q5_1)  // one lane per 32-block
        waves_k = (int)((p.nb + 63) / 64);
    else if (lut_type(p.wtype))  // one lane per 32 elements
        waves_k = (int)((p.K / 32 + 63) / 64);
    else if (k23_type(p.wtype))  // four lanes per super-block
        waves_k = (int)((p.nb + 15) / 16);
    else if (gemv_v2(p))
        waves_k = (int)((p.nb + 15) / 16);
    else
        waves_k = (int)((p.nb + 7) / 8);
    if (waves_k > 8) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: ne00 = %lld too large for the decode kernel", (long long)p.K);
    // K-quants (Q4_K, Q6_K): T row teams share one LDS copy of the quantized
    // activations; a team's wavefronts hold NG groups of RB rows in flight.
    const bool q4k = gemv_v2(p);
    int rb_d, ng_d, ns_d = 2, teams_d = p.N < 8192 && p.M <= 2 ? 4 : 8;
    gemv_groups(p.wtype, p.M, p.N, rb_d, ng_d);
    if (q4k && p.wtype == GHIP_TYPE_Q4_K && p.M <= 4 && waves_k == 1) {
        rb_d = 1;
        gemv_q4k_one_row(p.N, teams_d, ng_d, ns_d);
        // 3-4 rows: two one-row groups per team under 8192 rows; from 8192 rows
        // (3 rows there, 4 take the matrix-core kernel) groups of two rows
        // (4096 -> 14336 at 4 rows: 21.8 us one-row, 16.9 us two-row groups)
        if (p.M > 2) teams_d = 8, ng_d = 2, ns_d = 2, rb_d = p.N < 8192 ? 1 : 2;
    }
    // Q5_K (fused, one row): the same rule (4096 -> 14336 12.6 -> 9.7 us,
    // 4096 -> 4096 5.9 -> 5.0 us)
    if (q4k && p.wtype == GHIP_TYPE_Q5_K && p.M == 1 && fused && waves_k == 1) {
        rb_d = 1;
        gemv_q4k_one_row(p.N, teams_d, ng_d, ns_d);
    }
    // GHIP_GEMV_PERSIST=1: Q4_K at one row, K in one wavefront, from 8192
    // weight rows on the persistent grid (GHIP_GEMV_WGS workgroups of 8 teams,
    // each team an equal run of consecutive rows; "_r1x0").  Off by default:
    // 4096 -> 14336 measured 10.1 us at 256 or 512 workgroups (15.2 at 128)
    // against 9.8 us for the 448-workgroup grid.
    const bool persist = q4k && p.wtype == GHIP_TYPE_Q4_K && p.M == 1 && waves_k == 1 && fused && !sub &&
                         p.N >= 8192 && env_int("GHIP_GEMV_PERSIST", 0) != 0;
    const int rb = persist ? 1 : q4k ? env_int("GHIP_GEMV_RB", rb_d) : 8;
    const int ng = persist ? 0 : q4k ? env_int("GHIP_GEMV_NG", ng_d) : 1;
    if (q4k && !persist && !((rb == 2 && (ng == 2 || ng == 4 || ng == 8)) || (rb == 4 && (ng == 2 || ng == 4)) ||
                 (rb == 1 && p.wtype == GHIP_TYPE_Q4_K && p.M <= 4 && (ng == 2 || ng == 4 || ng == 7 || ng == 8)) ||
                 (rb == 1 && p.wtype == GHIP_TYPE_Q5_K && p.M == 1 && fused && (ng == 2 || ng == 4 || ng == 7 || ng == 8)) ||
                 (p.wtype == GHIP_TYPE_Q6_K && p.M == 1 && ((rb == 2 && ng == 8) || (rb == 1 && (ng == 4 || ng == 8))))))
        return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "GHIP_GEMV_RB x GHIP_GEMV_NG must be 2x2, 2x4, 2x8, 4x2 or 4x4");
    const int rows_per_team = rb * ng;
    // 8 teams, except 4 for one or two activation rows on matrices under 8192
    // rows: measured on 4096->1024 / 4096->4096 / 4096->14336 at batch 1-8
    // (there, fewer and fuller workgroups quantize the activation fewer times)
    const int teams = q4k ? std::max(1, std::min(8 / waves_k, env_int("GHIP_GEMV_TEAMS", teams_d))) : 1;
    const int rows_per_wg = persist ? 0 : rows_per_team * teams;
    const unsigned grid = persist ? (unsigned)std::max(1, std::min(env_int("GHIP_GEMV_WGS", 256), (int)((p.N + 7) / 8)))
                                  : (unsigned)((p.N + rows_per_wg - 1) / rows_per_wg);
    const int64_t cgrp = k23_type(p.wtype) ? 4 : 8;  // activation columns per launch
    for (int64_t c0 = 0; c0 < p.M; c0 += cgrp) {
        const int nc = (int)std::min<int64_t>(cgrp, p.M - c0);
        const int NC = nc == 1 ? 1 : nc == 2 ? 2 : nc <= 4 ? 4 : 8;
        std::string name = std::string(gemv_base(p.wtype)) + (p.wtype == GHIP_TYPE_Q6_K && q4k ? "_v2" : "") +
                           (fused ? "_f" : "") + (sub ? "_sub" : "") +
                           "_c" + std::to_string(NC) + (q4k ? "_r" + std::to_string(rb) + "x" + std::to_string(ng) : std::string());
        const bool one_row = q4k && !persist && rb == 1 &&
                             ((p.wtype == GHIP_TYPE_Q4_K && p.M <= 4) || (p.wtype == GHIP_TYPE_Q5_K && p.M == 1 && fused));
        const int ns = one_row ? env_int("GHIP_GEMV_NS", ns_d) : 2;
        // Q4_K names carry the slot count when it is not 2, Q5_K's one-row kernels always
        if (ns != 2 || (one_row && p.wtype == GHIP_TYPE_Q5_K)) name += "s" + std::to_string(ns);
        // Q4_0 in whole 8-row groups and block pairs, at most two columns: the
        // variant with unconditional loads, activations first (4096 x 4096,
        // fused: see gemv_q4_0_full_impl)
        if (p.wtype == GHIP_TYPE_Q4_0 && p.N % 8 == 0 && p.nb % 2 == 0 && NC <= 2 &&
            env_int("GHIP_GEMV_Q40_FULL", 1) != 0)
            name.replace(0, std::strlen("ghip_gemv_q4_0"), "ghip_gemv_q4_0_full");
        // Q5_0 from ready Q8_0 rows, the same conditions (4096 -> 14336:
        // 13.9 -> 11.95 us; Q8_0 keeps gemv_pair_q8_impl, slower this way)
        if (p.wtype == GHIP_TYPE_Q5_0 && !fused && p.N % 8 == 0 && p.nb % 2 == 0 && NC <= 2 &&
            env_int("GHIP_GEMV_Q40_FULL", 1) != 0)
            name.replace(0, std::strlen("ghip_gemv_q5_0"), "ghip_gemv_q5_0_full");
        int32_t *sub_c = sub;
        if (sub) {
            sub_c = sub + c0 * p.N * subsums_per_block(p.wtype) * p.nb;
        }
        ghip_status st;
        ctx->expect(dst + c0 * ldd, win2d(nc, ldd, p.N), "dst");
        if (sub) ctx->expect(sub_c, sub_bytes(p, nc), "sub-sums");
        if (q4k) {
            // LDS: codes [NC][K] | d [NC][nb] | 16-element sums [NC][nb][16] | partials
            const size_t shmem = (size_t)NC * p.K + (size_t)NC * p.nb * 4 + (size_t)NC * p.nb * 16 * 4 +
                                 (size_t)rows_per_wg * waves_k * NC * sizeof(float);
            if (shmem > 160 * 1024) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: decode LDS image too large");
            // (Q5_K: -1 selects the tiled kernel's fold, the reference's route from 8 rows)
            const int n_mat = p.wtype == GHIP_TYPE_Q5_K ? (p.M >= 8 ? -1 : 0)
                                                        : (int)std::max<int64_t>(0, std::min<int64_t>(nc, p.n_mat - c0));
            st = ctx->launch(name, dim3(grid), dim3(64 * waves_k * teams), shmem, s, (const uint8_t *)w,
                             (int64_t)p.w_row_bytes, (int)p.N, (int)p.nb, act + c0 * act_rb, (int64_t)act_rb, nc,
                             dst + c0 * ldd, (int64_t)ldd, sub_c, n_mat);
        } else {
            st = ctx->launch(name, dim3(grid), dim3(64 * waves_k), 0, s, (const uint8_t *)w, (int64_t)p.w_row_bytes,
                             (int)p.N, (int)p.nb, act + c0 * act_rb, (int64_t)act_rb, nc, dst + c0 * ldd,
                             (int64_t)ldd, sub_c);
        }
        if (st != GHIP_STATUS_SUCCESS) return st;
    }
    return GHIP_STATUS_SUCCESS;
}

// Prefill path (Q4_K, many activation rows): the Q8_K activations are laid
// out for the GEMM (codes | bsum16 | d, tokens padded to 128), then the int8
// MFMA GEMM runs on 128 x 128 tiles.
constexpr size_t kGemmSmem128 = 116224, kGemmSmem64 = 76544;  // sizeof(g3::Smem<BM>) in ghip_gemm.hip
constexpr size_t kGemmSmemQ6 = 152320;
constexpr size_t kGemmSmemQ8 = 22528;                          // sizeof(g8::Smem) in ghip_gemm.hip                         // sizeof(g6::Smem) in ghip_gemm.hip
constexpr size_t kGemmSmemW8 = 148480;  // 2 * sizeof(g4::Stage<256>) in ghip_gemm.hip
// GHIP_GEMM_BM=128 selects the 128 x 128 tiles of gemm_q4K_impl
int gemm_bm() { return env_int("GHIP_GEMM_BM", 64) == 128 ? 128 : 64; }
// Q4_K GEMM kernel: tile (tokens x rows), threads, LDS bytes
struct GemmKernel {
    const char *name, *name_sub, *name_multi;
    int bm, bn, threads;
    size_t smem;
};
const GemmKernel kGemmW8 = {"ghip_gemm_q4_K_w8", "ghip_gemm_q4_K_w8_sub", "ghip_gemm_q4_K_w8_multi", 128, 256, 512,
                            kGemmSmemW8};
const GemmKernel kGemmM64 = {"ghip_gemm_q4_K_m64", "ghip_gemm_q4_K_m64_sub", "ghip_gemm_q4_K_m64_multi", 64, 128, 256,
                             kGemmSmem64};
const GemmKernel kGemmM128 = {"ghip_gemm_q4_K", "ghip_gemm_q4_K_sub", nullptr, 128, 128, 512, kGemmSmem128};
// Q5_K: the wide tiles with the fifth-bit plane (ghip_gemm.hip gemm_q4K_wide_impl<8, _, true>)
const GemmKernel kGemmQ5W8 = {"ghip_gemm_q5_K_w8", "ghip_gemm_q5_K_w8_sub", nullptr, 128, 256, 512, kGemmSmemW8};
int64_t gemm_tiles(const GemmKernel &k, int64_t M, int64_t N) { return ((M + k.bm - 1) / k.bm) * ((N + k.bn - 1) / k.bn); }
// The wide 128 x 256 tiles (one workgroup of 8 wavefronts per CU) when they
// give at least half a wave of workgroups; otherwise 64 x 128 tiles (two per
// CU) with split K.  GHIP_GEMM_KERNEL=w8|m64|m128 forces one.
const GemmKernel &gemm_kernel(int64_t M, int64_t N) {
    const char *v = getenv("GHIP_GEMM_KERNEL");
    const std::string k = v ? v : "";
    if (k == "w8") return kGemmW8;
    if (k == "m64") return kGemmM64;
    if (k == "m128" || gemm_bm() == 128) return kGemmM128;
    return gemm_tiles(kGemmW8, M, N) >= 128 ? kGemmW8 : kGemmM64;
}
// K slices for grids that would leave CUs idle (fewer than 128 tiles); the
// slices' partial sums are added in order by ghip_gemm_splitk_reduce
const GemmKernel &gemm_kernel_for(const MulMatPlan &p) {
    return p.wtype == GHIP_TYPE_Q5_K ? kGemmQ5W8 : gemm_kernel(p.M, p.N);
}
int gemm_nsplit(const MulMatPlan &p) {
    const int64_t tiles = gemm_tiles(gemm_kernel_for(p), p.M, p.N);
    if (tiles >= 128 || p.N % 4) return 1;
    const int64_t want = (256 + tiles - 1) / tiles;
    const int64_t nbs = (p.nb + want - 1) / want;  // super-blocks per slice
    return (int)((p.nb + nbs - 1) / nbs);
}
// Q6_K prefill workspace: f16 codes [Mpad][K] | dT [nb][Mpad] | repacked weights [N][nb][336]
constexpr size_t kQ6R = 336;
// registered MXFP4 experts (ghip_mxfp4_repack): 128-row blocks, groups of 4
// 17-byte blocks, 80-byte windows -> one 10240-byte run per (expert, row block, group)
constexpr int64_t kMoeRows = 128, kMoeGroup = 4;
constexpr size_t kMoeWindowRun = 128 * 80;
size_t gemm_q6k_bytes(const MulMatPlan &p, size_t *codes_b, size_t *dt_b) {
    const size_t Mpad = (size_t)(p.M + 127) / 128 * 128, nbk = (size_t)p.K / 256;
    *codes_b = (Mpad * (size_t)p.K * 2 + 255) & ~(size_t)255;
    *dt_b = (nbk * Mpad * 4 + 255) & ~(size_t)255;
    return *codes_b + *dt_b + (size_t)p.N * nbk * kQ6R;
}
// Q4_0 / Q5_0 / Q8_0 prefill workspace: act codes [Mpad][Kpad] | da [nbp][Mpad] |
// weight codes [Npad][Kpad] | dw [nbp][Npad] (K padded to 128, rows to 128)
struct Q8Layout {
    int64_t Mpad, Npad, Kpad, nbp;
    size_t act_b, da_b, w_b, dw_b;
    size_t dsb_b;  // IQ4_XS: d per (super-block, row), after dw
};
Q8Layout q8_layout(int64_t M, int64_t N, int64_t K) {
    Q8Layout L;
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    L.Mpad = (M + 127) / 128 * 128;
    L.Npad = (N + 127) / 128 * 128;
    L.Kpad = (K + 127) / 128 * 128;
    L.nbp = L.Kpad / 32;
    L.act_b = up((size_t)L.Mpad * L.Kpad);
    L.da_b = up((size_t)L.nbp * L.Mpad * 4);
    L.w_b = up((size_t)L.Npad * L.Kpad);
    L.dw_b = up((size_t)L.nbp * L.Npad * 4);
    L.dsb_b = up((size_t)(L.Kpad / 256) * L.Npad * 4);
    return L;
}
// the GEMM's per-weight extra: IQ4_XS keeps its super-block scales apart
size_t q8_extra_b(int wtype, const Q8Layout &L) { return wtype == GHIP_TYPE_IQ4_XS ? L.dsb_b : 0; }
size_t gemm_layout_bytes(const MulMatPlan &p) {
    if (gemm_q8_family(p.wtype)) {
        const Q8Layout L = q8_layout(p.M, p.N, p.K);
        return L.act_b + L.da_b + L.w_b + L.dw_b + q8_extra_b(p.wtype, L);
    }
    if (p.wtype == GHIP_TYPE_Q6_K) {
        size_t a, b;
        return gemm_q6k_bytes(p, &a, &b);
    }
    const size_t Mpad = (size_t)(p.M + 127) / 128 * 128, nbk = (size_t)p.K / 256;
    const int ns = gemm_nsplit(p);
    const size_t part = ns > 1 ? (size_t)ns * (size_t)p.M * (size_t)p.N * 4 : 0;
    return ((Mpad * (size_t)p.K + nbk * Mpad * 32 + nbk * Mpad * 4 + 255) & ~(size_t)255) + part;
}
// Q6_K: repack the weights into aligned records, lay the codes out as f16, then
// the f16-MFMA GEMM on 64 x 128 tiles (one workgroup per CU, 137 KB of LDS)
// The Q6_K weights as the GEMM's 336-byte records: rebuilt into the
// workspace by every call, unless ghip_weight_register keeps a copy.
ghip_status q6k_repack(ghip_context *ctx, const void *w, int64_t row_bytes, int64_t N, int64_t nbk, uint8_t *rep,
                       hipStream_t s) {
    const int64_t nblk = N * nbk;  // four blocks per workgroup
    ctx->expect(rep, (size_t)nblk * kQ6R, "Q6_K repack");
    return ctx->launch("ghip_q6K_repack", dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, s, (const uint8_t *)w,
                       row_bytes, (int)N, (int)nbk, rep);
}
const uint8_t *registered_q6k(ghip_context *ctx, const MulMatPlan &p, const void *w) {
    auto it = ctx->wcache.find({w, GHIP_TYPE_Q6_K, p.K, p.N, 1, (uint64_t)p.w_row_bytes, 0});
    return it == ctx->wcache.end() ? nullptr : (const uint8_t *)it->second.p;
}
ghip_status run_gemm_q6k(ghip_context *ctx, const MulMatPlan &p, const void *w, const uint8_t *act,
                         const ghip_tensor *bf, float *dst, int64_t ldd, int32_t *sub, void *layout_ws, hipStream_t s) {
    size_t codes_b, dt_b;
    gemm_q6k_bytes(p, &codes_b, &dt_b);
    const int64_t Mpad = (p.M + 127) / 128 * 128, nbk = p.K / 256;
    uint16_t *codes = (uint16_t *)layout_ws;
    float *dT = (float *)((uint8_t *)layout_ws + codes_b);
    const uint8_t *rep = registered_q6k(ctx, p, w);
    ghip_status st = GHIP_STATUS_SUCCESS;
    if (!rep) {
        uint8_t *r = (uint8_t *)layout_ws + codes_b + dt_b;
        st = q6k_repack(ctx, w, p.w_row_bytes, p.N, nbk, r, s);
        if (st != GHIP_STATUS_SUCCESS) return st;
        rep = r;
    }
    ctx->expect(codes, (size_t)(Mpad * p.K * 2), "activation codes");
    ctx->expect(dT, (size_t)(nbk * Mpad * 4), "activation scales");
    if (bf)  // f32 activations: quantized straight into the layout
        st = ctx->launch("ghip_gemm_act_q8K_f16", dim3((unsigned)((p.M * nbk + 3) / 4)), dim3(256), 0, s,
                         (const float *)bf->data, (int64_t)bf->nb[1] / 4, (int)p.M, (int)Mpad, (int)nbk, (int)p.n_mat,
                         codes, dT);
    else
        st = ctx->launch("ghip_gemm_act_layout_f16", dim3((unsigned)((p.M * nbk + 3) / 4)), dim3(256), 0, s, act,
                         (int64_t)p.act_row_bytes, (int)p.M, (int)Mpad, (int)nbk, codes, dT);
    if (st != GHIP_STATUS_SUCCESS) return st;
    const unsigned grid = (unsigned)(((p.M + 63) / 64) * ((p.N + 127) / 128));
    ctx->expect(dst, win2d(p.M, ldd, p.N), "dst");
    if (sub) ctx->expect(sub, sub_bytes(p, p.M), "sub-sums");
    return ctx->launch(sub ? "ghip_gemm_q6_K_sub" : "ghip_gemm_q6_K", dim3(grid), dim3(256), kGemmSmemQ6, s,
                       (const uint8_t *)rep, (int)p.N, (int)nbk, (const uint16_t *)codes, (const float *)dT, (int)p.M,
                       (int)Mpad, dst, ldd, sub);
}

const char *q8w_repack_name(int wtype) {
    switch (wtype) {
    case GHIP_TYPE_Q4_0: return "ghip_gemm_q8w_repack_q4_0";
    case GHIP_TYPE_Q5_0: return "ghip_gemm_q8w_repack_q5_0";
    case GHIP_TYPE_IQ4_NL: return "ghip_gemm_q8w_repack_iq4_nl";
    case GHIP_TYPE_IQ4_XS: return "ghip_gemm_q8w_repack_iq4_xs";
    case GHIP_TYPE_Q1_0: return "ghip_gemm_q8w_repack_q1_0";
    case GHIP_TYPE_Q2_0: return "ghip_gemm_q8w_repack_q2_0";
    default: return "ghip_gemm_q8w_repack_q8_0";
    }
}
ghip_status q8w_repack(ghip_context *ctx, int wtype, const void *w, int64_t row_bytes, int64_t N, int64_t nb,
                       const Q8Layout &L, int8_t *codes, float *dw, hipStream_t s) {
    const int64_t n = L.Npad * L.nbp;
    ctx->expect(codes, (size_t)(L.Npad * L.Kpad), "weight codes");
    ctx->expect(dw, (size_t)(L.nbp * L.Npad * 4), "weight scales");
    if (wtype == GHIP_TYPE_IQ4_XS) ctx->expect((uint8_t *)dw + L.dw_b, (size_t)(L.Kpad / 256 * L.Npad * 4), "super-block scales");
    if (wtype == GHIP_TYPE_IQ4_XS)  // the super-block scales follow dw
        return ctx->launch(q8w_repack_name(wtype), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           (const uint8_t *)w, row_bytes, (int)N, (int)nb, (int)L.Kpad, (int)L.Npad, codes, dw,
                           (float *)((uint8_t *)dw + L.dw_b));
    return ctx->launch(q8w_repack_name(wtype), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       (const uint8_t *)w, row_bytes, (int)N, (int)nb, (int)L.Kpad, (int)L.Npad, codes, dw);
}
// Q4_0 / Q5_0 / Q8_0 from f32 rows: Q8_0 codes into the layout, the weights as
// int8 codes (kept if registered), then the int8-MFMA GEMM on 64 x 128 tiles
ghip_status run_gemm_q8(ghip_context *ctx, const MulMatPlan &p, const void *w, const ghip_tensor *bf, float *dst,
                        int64_t ldd, int32_t *sub, void *layout_ws, hipStream_t s) {
    const Q8Layout L = q8_layout(p.M, p.N, p.K);
    uint8_t *base = (uint8_t *)layout_ws;
    int8_t *ac = (int8_t *)base;
    float *da = (float *)(base + L.act_b);
    const int8_t *wc;
    const float *dw;
    auto it = ctx->wcache.find({w, p.wtype, p.K, p.N, 1, (uint64_t)p.w_row_bytes, 0});
    ghip_status st;
    if (it != ctx->wcache.end()) {
        wc = (const int8_t *)it->second.p;
        dw = (const float *)((const uint8_t *)it->second.p + L.w_b);
    } else {
        int8_t *c = (int8_t *)(base + L.act_b + L.da_b);
        float *d = (float *)(base + L.act_b + L.da_b + L.w_b);
        st = q8w_repack(ctx, p.wtype, w, p.w_row_bytes, p.N, p.nb, L, c, d, s);
        if (st != GHIP_STATUS_SUCCESS) return st;
        wc = c;
        dw = d;
    }
    const int64_t ablocks = L.Mpad * L.nbp;
    ctx->expect(ac, (size_t)(L.Mpad * L.Kpad), "activation codes");
    ctx->expect(da, (size_t)(L.nbp * L.Mpad * 4), "activation scales");
    const int nb32 = (int)(p.K / 32);  // the GEMM's blocks are 32 elements (Q8_0 activation blocks)
    if (p.wtype == GHIP_TYPE_IQ4_XS)  // Q8_K activations: codes and the block scale per 32-group
        st = ctx->launch("ghip_gemm_act_q8K_q8", dim3((unsigned)((L.Mpad * p.nb + 3) / 4)), dim3(256), 0, s,
                         (const float *)bf->data, (int64_t)bf->nb[1] / 4, (int)p.M, (int)L.Mpad, (int)p.nb,
                         (int)L.Kpad, ac, da);
    else
        st = ctx->launch("ghip_gemm_act_q8_0", dim3((unsigned)((ablocks * 8 + 255) / 256)), dim3(256), 0, s,
                         (const float *)bf->data, (int64_t)bf->nb[1] / 4, (int)p.M, (int)L.Mpad, nb32,
                         (int)L.Kpad, ac, da);
    if (st != GHIP_STATUS_SUCCESS) return st;
    const unsigned grid = (unsigned)(((p.M + 63) / 64) * ((p.N + 127) / 128));
    ctx->expect(dst, win2d(p.M, ldd, p.N), "dst");
    if (sub) ctx->expect(sub, sub_bytes(p, p.M), "sub-sums");
    if (p.wtype == GHIP_TYPE_IQ4_XS)
        return ctx->launch(sub ? "ghip_gemm_q8_xs_sub" : "ghip_gemm_q8_xs", dim3(grid), dim3(256), kGemmSmemQ8, s, wc,
                           dw, (int)p.N, (int)L.Npad, nb32, (int)L.Kpad, (const int8_t *)ac, (const float *)da,
                           (int)p.M, (int)L.Mpad, dst, ldd, sub, (const float *)((const uint8_t *)dw + L.dw_b));
    return ctx->launch(sub ? "ghip_gemm_q8_sub" : "ghip_gemm_q8", dim3(grid), dim3(256), kGemmSmemQ8, s, wc, dw,
                       (int)p.N, (int)L.Npad, nb32, (int)L.Kpad, (const int8_t *)ac, (const float *)da, (int)p.M,
                       (int)L.Mpad, dst, ldd, sub);
}

// act: Q8_K rows (bf == nullptr), or bf: the f32 activations, quantized
// straight into the GEMM layout
ghip_status run_gemm(ghip_context *ctx, const MulMatPlan &p, const void *w, const uint8_t *act, const ghip_tensor *bf,
                     float *dst, int64_t ldd, int32_t *sub, void *layout_ws, hipStream_t s) {
    if (p.wtype == GHIP_TYPE_Q6_K) return run_gemm_q6k(ctx, p, w, act, bf, dst, ldd, sub, layout_ws, s);
    if (gemm_q8_family(p.wtype)) return run_gemm_q8(ctx, p, w, bf, dst, ldd, sub, layout_ws, s);
    const int64_t Mpad = (p.M + 127) / 128 * 128, K = p.K, nbk = p.K / 256;
    int8_t *codes = (int8_t *)layout_ws;
    uint16_t *bsT = (uint16_t *)(codes + Mpad * K);
    float *dT = (float *)(bsT + nbk * Mpad * 16);
    const unsigned lgrid = (unsigned)((p.M * nbk + 3) / 4);
    ctx->expect(codes, (size_t)(Mpad * K), "activation codes");
    ctx->expect(bsT, (size_t)(nbk * Mpad * 32), "activation bsum16");
    ctx->expect(dT, (size_t)(nbk * Mpad * 4), "activation scales");
    ghip_status st =
        bf ? ctx->launch("ghip_gemm_act_q8K", dim3(lgrid), dim3(256), 0, s, (const float *)bf->data,
                         (int64_t)bf->nb[1] / 4, (int)p.M, (int)Mpad, (int)nbk, (int)p.n_mat, codes, bsT, dT)
           : ctx->launch("ghip_gemm_act_layout", dim3(lgrid), dim3(256), 0, s, act, (int64_t)p.act_row_bytes,
                         (int)p.M, (int)Mpad, (int)nbk, codes, bsT, dT);
    if (st != GHIP_STATUS_SUCCESS) return st;
    const GemmKernel &gk = gemm_kernel_for(p);
    const unsigned grid = (unsigned)gemm_tiles(gk, p.M, p.N);
    const int ns = gemm_nsplit(p);
    const int nbs = (int)((p.nb + ns - 1) / ns);
    float *part = ns > 1 ? (float *)((uint8_t *)layout_ws +
                                     (((size_t)Mpad * K + nbk * Mpad * 32 + nbk * Mpad * 4 + 255) & ~(size_t)255))
                         : dst;
    const int64_t zstride = ns > 1 ? p.M * p.N : 0;
    if (ns > 1) ctx->expect(part, (size_t)ns * (size_t)(p.M * p.N) * 4, "split-K partials");
    else ctx->expect(dst, win2d(p.M, ldd, p.N), "dst");
    if (sub) ctx->expect(sub, sub_bytes(p, p.M), "sub-sums");
    st = ctx->launch(sub ? gk.name_sub : gk.name, dim3(grid, ns), dim3(gk.threads), gk.smem, s,
                     (const uint8_t *)w, (int64_t)p.w_row_bytes, (int)p.N, (int)p.nb, (const int8_t *)codes,
                     (const uint16_t *)bsT, (const float *)dT, (int)p.M, (int)Mpad, part,
                     ns > 1 ? (int64_t)p.N : (int64_t)ldd, sub, nbs, zstride);
    if (st != GHIP_STATUS_SUCCESS || ns == 1) return st;
    const unsigned rgrid = (unsigned)((p.M * p.N / 4 + 255) / 256);
    ctx->expect(dst, win2d(p.M, ldd, p.N), "dst");
    return ctx->launch("ghip_gemm_splitk_reduce", dim3(rgrid), dim3(256), 0, s, (const float *)part, ns, (int)p.M,
                       (int)p.N, dst, (int64_t)ldd);
}

bool use_gemm(const MulMatPlan &p) {
    if (p.M > INT32_MAX) return false;
    if (p.wtype == GHIP_TYPE_Q4_K) return p.M >= env_int("GHIP_GEMM_MIN_ROWS", 16);
    // Q5_K: the wide Q4_K tiles with a fifth-bit plane, from 16 rows
    if (p.wtype == GHIP_TYPE_Q5_K) return p.M >= env_int("GHIP_GEMM_Q5K_MIN_ROWS", 16);
    // Q6_K: the f16-MFMA GEMM from 64 activation rows (below, the 8-column decode kernels)
    if (p.wtype == GHIP_TYPE_Q6_K) return p.M >= env_int("GHIP_GEMM_Q6K_MIN_ROWS", 64) && p.K >= 512;
    // Q4_0 / Q5_0 / Q8_0 from f32 activations: the int8-MFMA GEMM from 32 rows
    if (gemm_q8_family(p.wtype)) return !p.act_pre && p.M >= env_int("GHIP_GEMM_Q8_MIN_ROWS", 32);
    return false;
}
// the prefill GEMM (every GEMM also writes the sub-sums' layout)
bool gemm_route(const MulMatPlan &p, bool sub) {
    (void)sub;
    return use_gemm(p);
}

// workspace of one MUL_MAT: [quantized activations | GEMM layout | f32
// scratch output when only sub-sums are wanted]
size_t mul_mat_ws_bytes(const MulMatPlan &p, bool has_dst, bool act_out, size_t *act_b, size_t *lay_b,
                        bool sub = false) {
    if (dense_type(p.wtype)) {  // F32 / F16 / BF16 weights read src1 as it is
        if (act_b) *act_b = 0;
        if (lay_b) *lay_b = 0;
        return 0;
    }
    // (the GEMM quantizes f32 activations straight into its layout)
    const bool gemm = !act_out && gemm_route(p, sub);
    // (the split-K decode kernels quantize inside; their layout is the partials)
    const bool sk = !act_out && !gemm && use_sk(p);
    const size_t act_bytes = p.act_pre || gemm || sk ? 0 : ((size_t)(p.M * p.act_row_bytes) + 255) & ~(size_t)255;
    const size_t lay_bytes = gemm ? gemm_layout_bytes(p) : sk ? sk_part_bytes(p) : 0;
    if (act_b) *act_b = act_bytes;
    if (lay_b) *lay_b = lay_bytes;
    return (act_out ? 0 : act_bytes) + lay_bytes + (has_dst || act_out ? 0 : (size_t)(p.M * p.N * 4));
}

// F32 / F16 / BF16 weights: the dense decode kernel over groups of at most 8
// activation rows (compute.rs:1680-1745)
ghip_status run_dense(ghip_context *ctx, const MulMatPlan &p, const ghip_tensor *a, const ghip_tensor *b, float *dst,
                      int64_t ldd, hipStream_t s) {
    const char *tn = p.wtype == GHIP_TYPE_F32 ? "f32" : p.wtype == GHIP_TYPE_F16 ? "f16" : "bf16";
    // 16-byte chunks of 8 elements where every row starts 16-byte aligned
    const int esz = p.wtype == GHIP_TYPE_F32 ? 4 : 2;
    const int vec = p.K % 8 == 0 && (uintptr_t)a->data % 16 == 0 && p.w_row_bytes % 16 == 0 ? 1 : 0;
    (void)esz;
    const int64_t x_stride = (int64_t)b->nb[1] / 4;
    for (int64_t c0 = 0; c0 < p.M; c0 += 8) {
        const int nc = (int)std::min<int64_t>(8, p.M - c0);
        const int NC = nc == 1 ? 1 : nc == 2 ? 2 : nc <= 4 ? 4 : 8;
        const std::string name = std::string("ghip_gemv_dense_") + tn + "_c" + std::to_string(NC);
        ctx->expect(dst + c0 * ldd, win2d(nc, ldd, p.N), "dst");
        ghip_status st = ctx->launch(name, dim3((unsigned)((p.N + 7) / 8)), dim3(256), 0, s, (const uint8_t *)a->data,
                                     (int64_t)p.w_row_bytes, (int)p.N, (int)p.K, (const float *)b->data + c0 * x_stride,
                                     x_stride, nc, dst + c0 * ldd, ldd, vec);
        if (st != GHIP_STATUS_SUCCESS) return st;
    }
    return GHIP_STATUS_SUCCESS;
}

// one 2-D MUL_MAT (a single plane of src0, src1 and dst)
ghip_status mul_mat_plane(ghip_context *ctx, const ghip_tensor *a, const ghip_tensor *b, const ghip_tensor *d,
                          int32_t *sub, void *act_out, void *stream, void *fixed_ws, size_t fixed_bytes) {
    std::lock_guard<std::mutex> lock(ctx->mu);
    // a fixed scratch serves this call only
    struct CallScratch {
        ghip_context *c;
        CallScratch(ghip_context *c_, void *p, size_t n) : c(c_) { c->call_ws = p; c->call_ws_size = n; }
        ~CallScratch() { c->call_ws = nullptr; c->call_ws_size = 0; }
    } call_scratch(ctx, fixed_ws, fixed_bytes);
    MulMatPlan p;
    ghip_status st;
    if (!plan_mul_mat(ctx, a, b, d, p, st)) return st;
    hipStream_t s = (hipStream_t)stream;
    if (p.M == 0 || p.N == 0) return GHIP_STATUS_SUCCESS;  // empty operands: nothing to compute
    if (!ctx->set_device()) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    if (!d && !sub && !act_out) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: no output");
    st = ctx->begin(s);
    if (st != GHIP_STATUS_SUCCESS) return st;
    if (d) ctx->allow(d->data, win2d(p.M, (int64_t)d->nb[1], (int64_t)d->ne[0] * 4, 1), "dst");
    ctx->allow(sub, sub_bytes(p, p.M), "sub-sums");
    ctx->allow(act_out, (size_t)(p.M * p.act_row_bytes), "activation output");
    size_t act_bytes, lay_bytes;
    const size_t need = mul_mat_ws_bytes(p, d != nullptr, act_out != nullptr, &act_bytes, &lay_bytes, sub != nullptr);
    void *ws = nullptr;
    if (need) {
        st = ctx->workspace(need, s, &ws);
        if (st != GHIP_STATUS_SUCCESS) return st;
    }
    void *act = act_out ? act_out : ws;
    if (act_out) {
        if (dense_type(p.wtype)) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat_act: F32 / F16 / BF16 weights quantize nothing");
        if (p.act_pre) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat_act: src1 is already quantized");
        return quantize_act(ctx, p, b, act, s);
    }
    if (dense_type(p.wtype)) {
        if (sub || !d) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: F32 / F16 / BF16 weights have no integer sub-sums");
        return run_dense(ctx, p, a, b, (float *)d->data, (int64_t)d->nb[1] / 4, s);
    }
    void *lay = lay_bytes ? (void *)((uint8_t *)ws + act_bytes) : nullptr;
    float *dst = d ? (float *)d->data : (float *)((uint8_t *)ws + act_bytes + lay_bytes);
    // (GHIP_DEBUG_LDD_SKEW=k, dry-run contexts only: a deliberately wrong
    // leading dimension, the kind of host bug the store check exists for)
    const int64_t ldd = (d ? (int64_t)d->nb[1] / 4 : p.N) + (ctx->dry_run ? env_int("GHIP_DEBUG_LDD_SKEW", 0) : 0);
    if (gemm_route(p, sub != nullptr))
        return run_gemm(ctx, p, a->data, (const uint8_t *)b->data, p.act_pre ? nullptr : b, dst, ldd, sub, lay, s);
    if (use_sq(p)) {
        const uint8_t *a8 = (const uint8_t *)b->data;
        if (!p.act_pre) {
            st = quantize_act(ctx, p, b, act, s);
            if (st != GHIP_STATUS_SUCCESS) return st;
            a8 = (const uint8_t *)act;
        }
        SkLaunch g{};
        g.n = 1;
        g.m[0].W = (const uint8_t *)a->data;
        g.m[0].dst = dst;
        g.m[0].ldd = ldd;
        g.m[0].rows = (int)p.N;
        return launch_sq(ctx, p, g, a8, p.act_row_bytes, sub, s);
    }
    if (use_sk(p)) return run_sk(ctx, p, a->data, b, dst, ldd, sub, lay, s);
    if (p.act_pre) return run_gemv(ctx, p, a->data, (const uint8_t *)b->data, p.act_row_bytes, false, dst, ldd, sub, s);
    // Q8_0 quantization fused into the block-pair kernels for up to 4096 weight
    // rows: every workgroup then quantizes its lanes' blocks itself, which
    // beats a separate quantize launch there but adds more L2 reads and
    // per-wavefront work than it saves on larger matrices (4096x4096 Q4_0:
    // 7.25 -> 6.88 us; 4096->14336 Q5_0 / Q8_0: 13.9 -> 14.9 / 17.7 -> 18.2 us)
    const bool fuse_pair = gemv_pair(p.wtype) && p.N <= env_int("GHIP_GEMV_FUSE_MAX_ROWS", 4096);
    if ((gemv_v2(p) && !use_skinny(p)) || fuse_pair)  // quantization fused into the decode kernel
        return run_gemv(ctx, p, a->data, (const uint8_t *)b->data, (int64_t)b->nb[1], true, dst, ldd, sub, s);
    st = quantize_act(ctx, p, b, act, s);
    if (st != GHIP_STATUS_SUCCESS) return st;
    return run_gemv(ctx, p, a->data, (const uint8_t *)act, p.act_row_bytes, false, dst, ldd, sub, s);
}

// GGML_OP_MUL_MAT over batched operands (forward_mul_mat, compute.rs:1420-1450):
// plane (i12, i13) of dst is src0 plane (i12 / r2, i13 / r3) times src1 plane
// (i12, i13), each a 2-D MUL_MAT of its own (routes, quantization and the
// 4-row repack grouping are per plane, as in the reference's repack path,
// compute.rs:5346-5362).  Sub-sums and quantized activations of the planes
// follow one another in i13-major order.
ghip_status mul_mat_impl(ghip_context *ctx, const ghip_tensor *a, const ghip_tensor *b, const ghip_tensor *d,
                         int32_t *sub, void *act_out, void *stream, void *fixed_ws = nullptr, size_t fixed_bytes = 0) {
    if (!a || !b || (a->ne[2] == 1 && a->ne[3] == 1 && b->ne[2] == 1 && b->ne[3] == 1))
        return mul_mat_plane(ctx, a, b, d, sub, act_out, stream, fixed_ws, fixed_bytes);
    MulMatPlan p;
    ghip_status st;
    {
        std::lock_guard<std::mutex> lock(ctx->mu);
        if (!plan_mul_mat(ctx, a, b, d, p, st)) return st;
    }
    const int64_t r2 = b->ne[2] / a->ne[2], r3 = b->ne[3] / a->ne[3];
    const size_t sub_plane = (size_t)p.M * (size_t)p.N * (size_t)p.nb * (size_t)subsums_per_block(p.wtype);
    const size_t act_plane = (size_t)p.M * (size_t)p.act_row_bytes;
    int64_t plane = 0;
    for (int64_t i13 = 0; i13 < b->ne[3]; i13++)
        for (int64_t i12 = 0; i12 < b->ne[2]; i12++, plane++) {
            ghip_tensor a2 = *a, b2 = *b, d2;
            a2.data = (uint8_t *)a->data + (i12 / r2) * a->nb[2] + (i13 / r3) * a->nb[3];
            b2.data = (uint8_t *)b->data + i12 * b->nb[2] + i13 * b->nb[3];
            a2.ne[2] = a2.ne[3] = b2.ne[2] = b2.ne[3] = 1;
            if (d) {
                d2 = *d;
                d2.data = (uint8_t *)d->data + i12 * d->nb[2] + i13 * d->nb[3];
                d2.ne[2] = d2.ne[3] = 1;
            }
            st = mul_mat_plane(ctx, &a2, &b2, d ? &d2 : nullptr, sub ? sub + plane * sub_plane : nullptr,
                               act_out ? (uint8_t *)act_out + plane * act_plane : nullptr, stream, fixed_ws,
                               fixed_bytes);
            if (st != GHIP_STATUS_SUCCESS) return st;
        }
    return GHIP_STATUS_SUCCESS;
}

// ------------------------------------------------------------ FLASH_ATTN_EXT

// Mirror of FaParams in ghip_fa.hip (passed by value as the only kernel argument).
struct FaParams {
    const float *q;
    int64_t q_nb1, q_nb2;
    const uint16_t *k, *v;
    int64_t k_nb1, k_nb2, v_nb1, v_nb2;
    const uint16_t *mask;
    int64_t mask_nb1;
    int64_t mask_nb2;
    int mask_ne2;
    float *dst;
    float *part;
    const float *sinks;  // [H] or null
    int T, S, H, H_kv, nsplit, chunk;
    float scale, softcap, m0, m1;
    int n_head_log2;
    int DK, DV;
    int k_f32, v_f32;
    const uint8_t *mflags;
    int nqb, ntile;
    int direct;
};

float f32_param(const ghip_tensor *t, int i) {
    float f;
    memcpy(&f, &t->op_params[i], 4);
    return f;
}

bool plan_fa(ghip_context *ctx, const ghip_tensor *q, const ghip_tensor *k, const ghip_tensor *v,
             const ghip_tensor *mask, const ghip_tensor *sinks, const ghip_tensor *d, ghip_status &st) {
    st = GHIP_STATUS_BACKEND_ERROR;
    auto bad = [&](const char *why) { st = ctx->fail(GHIP_STATUS_BACKEND_ERROR, "flash_attn_ext: %s", why); return false; };
    if (!q || !k || !v || !d) return bad("null operand");
    if (q->type != GHIP_TYPE_F32 || q->nb[0] != 4) return bad("q must be F32 with nb0 == 4 (flash_attn.rs:322)");
    auto kv_ok = [](const ghip_tensor *t) {
        return (t->type == GHIP_TYPE_F16 && t->nb[0] == 2) || (t->type == GHIP_TYPE_F32 && t->nb[0] == 4);
    };
    if (!kv_ok(k) || !kv_ok(v)) return bad("k and v must be F16 or F32 rows (flash_attn.rs:305-313)");
    if (k->ne[0] != q->ne[0]) return bad("DK of q and k differ");
    if (k->ne[0] < 1 || k->ne[0] > 256 || v->ne[0] < 1 || v->ne[0] > 256) return bad("head sizes must be 1..256");
    // sequences (dim 3): q, k and v agree (flash_attn.rs:298); ghip_flash_attn_ext
    // runs them one by one
    if (q->ne[3] < 1 || k->ne[3] != q->ne[3] || v->ne[3] != q->ne[3]) return bad("ne3 of q, k and v differ");
    if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2]) return bad("k/v shapes differ");
    if (q->ne[2] % k->ne[2]) return bad("H % H_kv != 0");
    if (k->nb[1] % k->nb[0] || k->nb[2] % k->nb[0] || v->nb[1] % v->nb[0] || v->nb[2] % v->nb[0] || q->nb[1] % 4 ||
        q->nb[2] % 4)
        return bad("strides must be element multiples");
    if (mask) {
        if (mask->type != GHIP_TYPE_F16 || mask->nb[0] != 2) return bad("mask must be F16 rows (ggml.c:5515)");
        if (mask->ne[0] < k->ne[1] || mask->ne[1] < q->ne[1]) return bad("mask smaller than [S, T]");
        // planes broadcast to heads by h % ne2 and to sequences by i3 % ne3
        // (ggml.c:5517-5518, flash_attn.rs:30-37)
        if (mask->ne[2] < 1 || mask->ne[3] < 1 || q->ne[2] % mask->ne[2] || q->ne[3] % mask->ne[3])
            return bad("mask planes must divide the heads (ne2) and sequences (ne3)");
        if (mask->nb[1] % 2 || mask->nb[2] % 2) return bad("mask strides must be element multiples");
        if ((uint64_t)q->ne[1] * mask->nb[1] >= (1ull << 31)) return bad("mask spans >= 2 GiB");
    }
    if (sinks && (sinks->type != GHIP_TYPE_F32 || sinks->ne[0] < q->ne[2])) return bad("sinks must be F32 [H]");
    if (d->type != GHIP_TYPE_F32 || d->ne[0] != v->ne[0] || d->ne[1] != q->ne[2] || d->ne[2] != q->ne[1] ||
        d->ne[3] != q->ne[3] || d->nb[0] != 4 || d->nb[1] != (uint64_t)(4 * d->ne[0]) ||
        d->nb[2] != (uint64_t)(4 * d->ne[0] * d->ne[1]) || d->nb[3] % 4)
        return bad("dst must be F32 [DV, H, T, ne3], each sequence contiguous");
    if (q->ne[1] > INT32_MAX || k->ne[1] > INT32_MAX) return bad("dimension too large");
    // the kernels address one KV head with 32-bit byte offsets
    if ((uint64_t)k->ne[1] * std::max(k->nb[1], v->nb[1]) >= (1ull << 31)) return bad("a KV head spans >= 2 GiB");
    st = GHIP_STATUS_SUCCESS;
    return true;
}


// Launch geometry and workspace (split partials) of one FLASH_ATTN_EXT.
struct FaLayout {
    int G, QS, qtiles, nsplit, chunk;
    size_t ws_bytes;
    // prefill with a mask: the mask tile classes (ghip_fa_mask_scan) after the partials
    size_t flags_off;
    int nqb, ntile;
};
FaLayout fa_layout(int D, int T, int H, int S, int H_kv, int mask_planes = 0) {
    FaLayout L;
    // prefill workgroups hold G * QS wavefronts (G = H / H_kv heads times QS
    // query tiles of 32) so that every staged K/V tile serves >= 4 of them
    L.G = H / H_kv;
    const int W = std::max(4, std::min(8, env_int("GHIP_FA_WAVES", 4)));
    L.QS = std::max((4 + L.G - 1) / L.G, std::min((W + L.G - 1) / L.G, 8 / L.G));
    L.qtiles = (T + 32 * L.QS - 1) / (32 * L.QS);
    if (T == 1 && S >= 512) {
        // single-query split-KV route: enough key slices to give every CU
        // several workgroups
        int ns = std::max(1, std::min((S + 127) / 128, (env_int("GHIP_FA_DECODE_WGS", 512) + H_kv - 1) / H_kv));
        const int ch = (S + ns - 1) / ns;
        ns = std::max(1, (S + ch - 1) / ch);
        L.nsplit = ns;
        L.chunk = ch;
        L.ws_bytes = (size_t)H * ns * (2 + D) * sizeof(float);
        return L;
    }
    // slices of the KV range: enough workgroups to fill the GPU, 64-key multiples
    const int max_split = std::max(1, (S + 63) / 64);
    int nsplit = std::max(1, std::min(max_split, (env_int("GHIP_FA_WGS", 512) + L.qtiles * H_kv - 1) / (L.qtiles * H_kv)));
    int chunk = ((S + nsplit - 1) / nsplit + 63) / 64 * 64;
    if (chunk == 0) chunk = 64;
    nsplit = std::max(1, (S + chunk - 1) / chunk);
    L.nsplit = nsplit;
    L.chunk = chunk;
    const bool rowseq = T < 64 && !env_int("GHIP_FA_FORCE_MFMA", 0);  // one_chunk walk: no partials
    L.ws_bytes = rowseq ? 0 : (size_t)T * H * nsplit * (2 + D) * sizeof(float);
    L.nqb = (T + 31) / 32;
    L.ntile = (S + 63) / 64;
    L.flags_off = (L.ws_bytes + 255) & ~(size_t)255;
    if (!rowseq && mask_planes > 0 && env_int("GHIP_FA_MASK_SCAN", 1) != 0)
        L.ws_bytes = L.flags_off + (size_t)mask_planes * L.nqb * L.ntile;
    return L;
}

// ------------------------------------------------------------ MUL_MAT_ID

// MXFP4 expert kernel: the scaled-FP4 one (32-pair tiles) unless
// GHIP_MOE_KERNEL=f16 asks for the f16 one
bool moe_fp4(int tp) {
    const char *v = getenv("GHIP_MOE_KERNEL");
    (void)tp;
    return !(v && strcmp(v, "f16") == 0);
}

struct MoePlan {
    int wtype;  // MXFP4, Q4_K / Q5_K / Q6_K experts, or a type of the per-pair decode route
    bool generic;  // per-pair decode kernels (mmid_generic_type)
    int64_t K, rows, n_as, ne11, n_tokens, n_ids, nb;
    int64_t act_row_bytes;
};

// expert types that MUL_MAT_ID runs through the decode kernels, one (token,
// slot) pair per grid row (every type with a vec_dot_type, compute.rs:1926-1929)
const char *mmid_kernel_type(int t) {
    switch (t) {
    case GHIP_TYPE_Q4_0: return "q4_0";
    case GHIP_TYPE_Q5_0: return "q5_0";
    case GHIP_TYPE_Q8_0: return "q8_0";
    case GHIP_TYPE_Q4_1: return "q4_1";
    case GHIP_TYPE_Q5_1: return "q5_1";
    case GHIP_TYPE_Q2_K: return "q2_K";
    case GHIP_TYPE_Q3_K: return "q3_K";
    case GHIP_TYPE_IQ4_NL: return "iq4_nl";
    case GHIP_TYPE_IQ4_XS: return "iq4_xs";
    case GHIP_TYPE_NVFP4: return "nvfp4";
    case GHIP_TYPE_Q1_0: return "q1_0";
    case GHIP_TYPE_IQ2_XXS: return "iq2_xxs";
    case GHIP_TYPE_IQ2_XS: return "iq2_xs";
    case GHIP_TYPE_IQ2_S: return "iq2_s";
    case GHIP_TYPE_IQ3_XXS: return "iq3_xxs";
    case GHIP_TYPE_IQ3_S: return "iq3_s";
    case GHIP_TYPE_IQ1_S: return "iq1_s";
    case GHIP_TYPE_IQ1_M: return "iq1_m";
    default: return "q2_0";
    }
}
int mmid_act_type(int t) {
    if (t == GHIP_TYPE_Q4_1 || t == GHIP_TYPE_Q5_1) return GHIP_TYPE_Q8_1;
    if (t == GHIP_TYPE_Q2_K || t == GHIP_TYPE_Q3_K || t == GHIP_TYPE_IQ4_XS || grid_type(t)) return GHIP_TYPE_Q8_K;
    return GHIP_TYPE_Q8_0;
}
bool mmid_generic_type(int t) {
    return t == GHIP_TYPE_Q4_0 || t == GHIP_TYPE_Q5_0 || t == GHIP_TYPE_Q8_0 || t == GHIP_TYPE_Q4_1 ||
           t == GHIP_TYPE_Q5_1 || t == GHIP_TYPE_Q2_K || t == GHIP_TYPE_Q3_K || t == GHIP_TYPE_IQ4_NL ||
           t == GHIP_TYPE_IQ4_XS || t == GHIP_TYPE_NVFP4 || t == GHIP_TYPE_Q1_0 || t == GHIP_TYPE_Q2_0 || grid_type(t);
}
// forward_mul_mat_id (compute.rs:1917-2202): MXFP4, Q4_K, Q5_K and Q6_K experts on
// their own kernels, every other type with a vec_dot (compute.rs:1926-1929) on
// its decode kernel per (token, slot) pair.
bool plan_moe(ghip_context *ctx, const ghip_tensor *as, const ghip_tensor *b, const ghip_tensor *ids,
              const ghip_tensor *d, MoePlan &p, ghip_status &st) {
    st = GHIP_STATUS_BACKEND_ERROR;
    auto bad = [&](const char *why) { st = ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat_id: %s", why); return false; };
    if (!as || !b || !ids) return bad("null operand");
    p.wtype = as->type;
    p.generic = mmid_generic_type(p.wtype);
    if (p.wtype != GHIP_TYPE_MXFP4 && p.wtype != GHIP_TYPE_Q4_K && p.wtype != GHIP_TYPE_Q5_K &&
        p.wtype != GHIP_TYPE_Q6_K && !p.generic)
        return bad("experts must be MXFP4, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS, "
                   "NVFP4, Q1_0, Q2_0, IQ1_S, IQ1_M, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS or IQ3_S");
    const TypeInfo ti = type_info(p.wtype);
    if (as->ne[0] % ti.blck || as->ne[0] <= 0) return bad("ne00 must be a positive multiple of the block size");
    p.K = as->ne[0];
    p.rows = as->ne[1];
    p.n_as = as->ne[2];
    p.nb = p.K / ti.blck;
    if (as->ne[3] != 1) return bad("4-D experts are not supported");
    if (as->nb[0] != (uint64_t)ti.bytes || as->nb[1] != (uint64_t)(p.nb * ti.bytes) ||
        as->nb[2] < (uint64_t)(p.rows * p.nb * ti.bytes))
        return bad("expert rows must be contiguous blocks");
    if (b->type != GHIP_TYPE_F32 || b->nb[0] != 4 || b->ne[0] != p.K) return bad("b must be F32 [ne00, ...]");
    p.ne11 = b->ne[1];
    p.n_tokens = b->ne[2];
    if (b->ne[3] != 1 || b->nb[1] % 4 || b->nb[2] != b->nb[1] * (uint64_t)p.ne11)
        return bad("b must be [ne00, ne11, n_tokens] with rows at a uniform stride");
    if (ids->type != GHIP_TYPE_I32 || ids->nb[0] != 4 || ids->nb[1] % 4) return bad("ids must be I32 rows");
    p.n_ids = ids->ne[0];
    if (ids->ne[1] != p.n_tokens) return bad("ids->ne[1] != b->ne[2]");
    if (p.ne11 < 1 || p.ne11 > p.n_ids) return bad("need 1 <= ne11 <= n_ids (ggml.c mul_mat_id)");
    if (p.n_as < 1 || p.n_as > 4096) return bad("n_as out of range");
    if (p.n_ids * p.n_tokens > (1 << 24) || p.rows > INT32_MAX) return bad("too many (token, slot) pairs");
    if (d && (d->type != GHIP_TYPE_F32 || d->nb[0] != 4 || d->ne[0] != p.rows || d->ne[1] != p.n_ids ||
              d->ne[2] != p.n_tokens))
        return bad("dst must be F32 [rows, n_ids, n_tokens]");
    if (p.wtype != GHIP_TYPE_MXFP4 && p.nb > INT32_MAX / 256) return bad("ne00 too large");
    p.act_row_bytes = p.wtype == GHIP_TYPE_MXFP4 ? p.nb * 34 : p.nb * 292;
    if (p.generic) {  // the vec_dot_type's rows (vec_dot.rs:1727-1749)
        const int at = mmid_act_type(p.wtype);
        p.act_row_bytes = at == GHIP_TYPE_Q8_K ? p.K / 256 * 292 : at == GHIP_TYPE_Q8_1 ? p.K / 32 * 36 : p.K / 32 * 34;
    }
    st = GHIP_STATUS_SUCCESS;
    return true;
}

// MUL_MAT_ID workspace: Q8_0 rows | f16 slot codes | f32 scales | routing
// table | scratch output (sub-sums only)
struct MoeWs {
    int tp;
    int64_t max_tiles;
    size_t act, actf, actd, route, out, total;
};
MoeWs moe_ws(const MoePlan &p, bool has_dst, bool sub) {
    MoeWs L;
    const int64_t n_pairs = p.n_ids * p.n_tokens;
    // 32-pair tiles when experts see few pairs each (decode, small batches)
    const int tile_env = env_int("GHIP_MOE_TILE", 0);
    L.tp = (sub || tile_env == 32) ? 32 : tile_env == 64 ? 64 : n_pairs <= 48 * p.n_as ? 32 : 64;
    L.max_tiles = (n_pairs + L.tp - 1) / L.tp + p.n_as;
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    L.act = up((size_t)(p.ne11 * p.n_tokens * p.act_row_bytes));
    const bool kq = p.wtype != GHIP_TYPE_MXFP4;  // K-quants read the Q8_K rows directly
    if (kq) L.tp = 32;  // the K-quant kernel takes 32-pair tiles
    L.max_tiles = (n_pairs + L.tp - 1) / L.tp + p.n_as;
    L.actf = kq ? 0 : up((size_t)n_pairs * p.nb * 64);  // per routed pair
    L.actd = kq ? 0 : up((size_t)n_pairs * p.nb * 4);
    L.route = up((size_t)(2 + n_pairs + 3 * L.max_tiles) * 4);
    L.out = has_dst ? 0 : (size_t)(n_pairs * p.rows * 4);
    L.total = L.act + L.actf + L.actd + L.route + L.out;
    return L;
}

// The further expert types: every src1 row quantized to the vec_dot type
// (the wdata pass, compute.rs:1950-1976), then the decode kernel of each
// pair's expert on its row (grid: 8-row blocks x pairs).
ghip_status mul_mat_id_generic(ghip_context *ctx, const MoePlan &p, const ghip_tensor *as, const ghip_tensor *b,
                               const ghip_tensor *ids, const ghip_tensor *d, int32_t *sub, hipStream_t s) {
    const int64_t n_pairs = p.n_ids * p.n_tokens, act_rows = p.ne11 * p.n_tokens;
    const size_t act_b = ((size_t)(act_rows * p.act_row_bytes) + 255) & ~(size_t)255;
    const size_t out_b = d ? 0 : (size_t)(n_pairs * p.rows * 4);
    void *ws = nullptr;
    ghip_status st = ctx->workspace(act_b + out_b, s, &ws);
    if (st != GHIP_STATUS_SUCCESS) return st;
    uint8_t *act = (uint8_t *)ws;
    float *dst = d ? (float *)d->data : (float *)((uint8_t *)ws + act_b);
    const int64_t dst_nb1 = d ? (int64_t)d->nb[1] / 4 : p.rows;
    const int64_t dst_nb2 = d ? (int64_t)d->nb[2] / 4 : p.rows * p.n_ids;
    const int at = mmid_act_type(p.wtype);
    const int64_t x_stride = (int64_t)b->nb[1] / 4;
    ctx->expect(act, (size_t)(act_rows * p.act_row_bytes), "quantized activations");
    if (at == GHIP_TYPE_Q8_K)
        st = ctx->launch("ghip_quantize_q8_K", dim3((unsigned)((act_rows * (p.K / 256) + 3) / 4)), dim3(256), 0, s,
                         (const float *)b->data, x_stride, p.K, act_rows, act, p.act_row_bytes, (int64_t)0);
    else
        st = ctx->launch(at == GHIP_TYPE_Q8_1 ? "ghip_quantize_q8_1" : "ghip_quantize_q8_0",
                         dim3((unsigned)((act_rows * (p.K / 32) * 8 + 255) / 256)), dim3(256), 0, s,
                         (const float *)b->data, x_stride, p.K, act_rows, act, p.act_row_bytes);
    if (st != GHIP_STATUS_SUCCESS) return st;
    // the decode kernels' wavefronts per row (as run_gemv)
    int waves_k;
    if (gemv_pair(p.wtype)) waves_k = (int)(((p.nb + 1) / 2 + 63) / 64);
    else if (p.wtype == GHIP_TYPE_Q4_1 || p.wtype == GHIP_TYPE_Q5_1) waves_k = (int)((p.nb + 63) / 64);
    else if (lut_type(p.wtype)) waves_k = (int)((p.K / 32 + 63) / 64);
    else waves_k = (int)((p.nb + 15) / 16);  // Q2_K / Q3_K: four lanes per super-block
    if (waves_k > 8) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat_id: ne00 = %lld too large for the decode kernel", (long long)p.K);
    const int64_t sub_pair = p.rows * p.nb * subsums_per_block(p.wtype);
    if (sub) ctx->expect(sub, (size_t)(n_pairs * sub_pair * 4), "sub-sums");
    ctx->expect(dst, (size_t)((p.n_tokens - 1) * dst_nb2 + (p.n_ids - 1) * dst_nb1 + p.rows) * 4, "dst");
    const char *tn = mmid_kernel_type(p.wtype);
    const std::string name = std::string("ghip_mmid_gemv_") + tn + (sub ? "_sub" : "");
    constexpr int kRows = 8;  // weight rows per decode workgroup
    return ctx->launch(name, dim3((unsigned)((p.rows + kRows - 1) / kRows), (unsigned)n_pairs), dim3(64 * waves_k), 0,
                       s, (const uint8_t *)as->data, (int64_t)as->nb[1], (int64_t)as->nb[2], (int)p.rows, (int)p.nb,
                       (const uint8_t *)act, p.act_row_bytes, (int)p.ne11, (const int32_t *)ids->data,
                       (int64_t)ids->nb[1] / 4, (int)p.n_ids, (int)p.n_as, dst, dst_nb1, dst_nb2, sub, sub_pair,
                       kRows);
}

// Q8_0 activations, routing, then the tiled MFMA kernel; pairs with an
// invalid expert id get NaN rows (the reference asserts on them).
ghip_status mul_mat_id_impl(ghip_context *ctx, const ghip_tensor *as, const ghip_tensor *b, const ghip_tensor *ids,
                            const ghip_tensor *d, int32_t *sub, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    std::lock_guard<std::mutex> lock(ctx->mu);
    MoePlan p;
    ghip_status st;
    if (!plan_moe(ctx, as, b, ids, d, p, st)) return st;
    const int64_t n_pairs = p.n_ids * p.n_tokens;
    if (n_pairs == 0 || p.rows == 0) return GHIP_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;
    if (!ctx->set_device()) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    st = ctx->begin(s);
    if (st != GHIP_STATUS_SUCCESS) return st;
    if (d)
        ctx->allow(d->data, (size_t)((p.n_tokens - 1) * d->nb[2] + (p.n_ids - 1) * d->nb[1]) + (size_t)p.rows * 4, "dst");
    ctx->allow(sub, (size_t)(n_pairs * p.rows * p.nb * (p.wtype == GHIP_TYPE_MXFP4 ? 1 : subsums_per_block(p.wtype))) * 4,
               "sub-sums");
    if (p.generic) return mul_mat_id_generic(ctx, p, as, b, ids, d, sub, s);
    const MoeWs L = moe_ws(p, d != nullptr, sub != nullptr);
    const int tp = L.tp;
    const int64_t max_tiles = L.max_tiles;
    const int64_t act_rows = p.ne11 * p.n_tokens;
    const size_t act_bytes = L.act, actf_bytes = L.actf, actd_bytes = L.actd, route_bytes = L.route;
    void *ws = nullptr;
    st = ctx->workspace(L.total, s, &ws);
    if (st != GHIP_STATUS_SUCCESS) return st;
    uint8_t *act = (uint8_t *)ws;
    uint16_t *actf = (uint16_t *)((uint8_t *)ws + act_bytes);  // f16 codes
    float *actd = (float *)((uint8_t *)actf + actf_bytes);
    int32_t *route = (int32_t *)((uint8_t *)actd + actd_bytes);
    float *dst = d ? (float *)d->data : (float *)((uint8_t *)route + route_bytes);
    const int64_t dst_nb1 = d ? (int64_t)d->nb[1] / 4 : p.rows;
    const int64_t dst_nb2 = d ? (int64_t)d->nb[2] / 4 : p.rows * p.n_ids;
    const bool kq = p.wtype != GHIP_TYPE_MXFP4;
    if (kq) {  // quantize_row_q8_K for every src1 row (the wdata pass, compute.rs:1950-1976)
        const unsigned qgrid = (unsigned)((act_rows * p.nb + 3) / 4);
        st = ctx->launch("ghip_quantize_q8_K", dim3(qgrid), dim3(256), 0, s, (const float *)b->data,
                         (int64_t)b->nb[1] / 4, p.K, act_rows, act, p.act_row_bytes, (int64_t)0);
    } else if (!moe_fp4(tp)) {  // the f16 kernel's activation pass reads Q8_0 rows
        const unsigned qgrid = (unsigned)((act_rows * p.nb * 8 + 255) / 256);
        st = ctx->launch("ghip_quantize_q8_0", dim3(qgrid), dim3(256), 0, s, (const float *)b->data,
                         (int64_t)b->nb[1] / 4, p.K, act_rows, act, p.act_row_bytes);
    }
    if (st != GHIP_STATUS_SUCCESS) return st;
    const int64_t ids_nb1 = (int64_t)ids->nb[1] / 4;
    st = ctx->launch("ghip_moe_route", dim3(1), dim3(1024), (unsigned)(2 * p.n_as * 4), s, (const int32_t *)ids->data,
                     ids_nb1, (int)p.n_ids, (int)p.n_tokens, (int)p.n_as, route, (int)max_tiles, tp, dst, dst_nb1,
                     dst_nb2, (int)p.rows);
    if (st != GHIP_STATUS_SUCCESS) return st;
    if (kq) {
        const char *tn = p.wtype == GHIP_TYPE_Q4_K ? "q4_K" : p.wtype == GHIP_TYPE_Q5_K ? "q5_K" : "q6_K";
        const std::string name = std::string("ghip_mmid_") + tn + (sub ? "_sub" : "");
        const dim3 grid((unsigned)max_tiles, (unsigned)((p.rows + 15) / 16));
        return ctx->launch(name, grid, dim3(256), 0, s, (const uint8_t *)as->data, (int64_t)as->nb[1],
                           (int64_t)as->nb[2], (const uint8_t *)act, p.act_row_bytes, (int)p.ne11,
                           (const int32_t *)route, (int)n_pairs, (int)p.n_ids, dst, dst_nb1, dst_nb2, (int)p.rows,
                           (int)p.nb, sub);
    }
    // The scaled-FP4 kernel (FP8 planes of the codes), or with GHIP_MOE_KERNEL=f16
    // the f16 kernel (f16 codes); both write 64 bytes per routed pair and block
    const bool fp4 = moe_fp4(tp);
    const unsigned fgrid = (unsigned)((n_pairs * p.nb * 4 + 255) / 256);
    if (fp4)  // FP8 planes quantized straight from the f32 rows (no Q8_0 pass)
        st = ctx->launch("ghip_moe_act_fp8_f", dim3(fgrid), dim3(256), 0, s, (const float *)b->data,
                         (int64_t)b->nb[1] / 4, (int64_t)b->nb[2] / 4, (const int32_t *)route, (int)n_pairs,
                         (int)p.n_ids, (int)p.ne11, (int)p.nb, actf, actd);
    else
        st = ctx->launch("ghip_moe_act_f16", dim3(fgrid), dim3(256), 0, s, (const uint8_t *)act, p.act_row_bytes,
                         (const int32_t *)route, (int)n_pairs, (int)p.n_ids, (int)p.ne11, (int)p.nb, actf, actd);
    if (st != GHIP_STATUS_SUCCESS) return st;
    const bool repack = p.rows % 8 == 0;  // compute.rs:1965-1972 routes rows % 8 == 0 through the repack kernel
    std::string name = fp4 ? std::string("ghip_moe_fp4") + (tp == 64 ? "_t64" : "") + (repack ? "" : "_plain") +
                                 (sub ? "_sub" : "")
                           : std::string("ghip_moe_mxfp4_t") + (tp == 32 ? "32" : "64") + (repack ? "" : "_plain") +
                                 (sub ? "_sub" : "");
    // the scaled-FP4 kernel remaps its ids per XCD when the grid is a multiple of 8
    // (tiles past the route's count exit at once); GHIP_MOE_ORDER 0 / 1 / 2:
    // no remap / tiles fastest (default) / row blocks fastest
    const dim3 grid((unsigned)(fp4 ? (max_tiles + 7) / 8 * 8 : max_tiles), (unsigned)((p.rows + 127) / 128));
    if (fp4) {
        // the registered copy of the experts, if any (ghip_weight_register)
        // (used from GHIP_MOE_REG_MIN_ROWS weight rows: measured on the
        // gpt-oss-20b shapes, K = 2880, gate_up 5760 rows 129 us registered
        // against 167 us in the GGUF layout, down 2880 rows 129 against 92 us)
        auto it = ctx->wcache.find(ghip_context::key_of(as));
        const uint8_t *wrep = it == ctx->wcache.end() || p.rows < env_int("GHIP_MOE_REG_MIN_ROWS", 4096)
                                  ? nullptr : (const uint8_t *)it->second.p;
        const int ngp = (int)((p.nb + kMoeGroup - 1) / kMoeGroup);
        if (wrep) name += "_reg";
        return ctx->launch(name.c_str(), grid, dim3(256), 0, s, (const uint8_t *)as->data, (int64_t)as->nb[1],
                           (int64_t)as->nb[2], (const uint16_t *)actf, (const float *)actd, (int)p.ne11,
                           (const int32_t *)route, (int)n_pairs, (int)p.n_ids, dst, dst_nb1, dst_nb2, (int)p.rows,
                           (int)p.nb, sub, wrep, ngp, env_int("GHIP_MOE_ORDER", 1));
    }
    return ctx->launch(name.c_str(), grid, dim3(256), 0, s, (const uint8_t *)as->data, (int64_t)as->nb[1],
                       (int64_t)as->nb[2], (const uint16_t *)actf, (const float *)actd, (int)p.ne11,
                       (const int32_t *)route, (int)n_pairs, (int)p.n_ids, dst, dst_nb1, dst_nb2, (int)p.rows,
                       (int)p.nb, sub);
}

// ------------------------------------------------------------ graph compute

// Host mirror of GemvMulti in ghip_gemv.hip (kernel argument by value).
struct GemvMulti {
    const uint8_t *W[4];
    float *dst[4];
    int64_t ldd[4];
    int rows[4];
    int wg0[4];
    int n;
};

// [first, last) byte range a tensor's elements span (dims with ne > 1)
void byte_span(const ghip_tensor *t, uintptr_t &lo, uintptr_t &hi) {
    const TypeInfo ti = type_info(t->type);
    uint64_t ext = (uint64_t)(t->ne[0] / std::max(1, ti.blck)) * (uint64_t)ti.bytes;
    for (int d = 1; d < 4; d++)
        if (t->ne[d] > 1) ext += (uint64_t)(t->ne[d] - 1) * t->nb[d];
    lo = (uintptr_t)t->data;
    hi = lo + ext;
}
bool overlaps(const ghip_tensor *a, const ghip_tensor *b) {
    if (!a || !b) return false;
    uintptr_t alo, ahi, blo, bhi;
    byte_span(a, alo, ahi);
    byte_span(b, blo, bhi);
    return alo < bhi && blo < ahi;
}
bool same_view(const ghip_tensor *a, const ghip_tensor *b) {
    if (a->data != b->data || a->type != b->type) return false;
    for (int d = 0; d < 4; d++)
        if (a->ne[d] != b->ne[d] || a->nb[d] != b->nb[d]) return false;
    return true;
}
// a MUL_MAT node the multi-matrix kernels take: K-quant weights, 1-8 F32
// activation rows (Q6_K: one), a destination, the default 2x2 row groups
bool multi_candidate(const ghip_node &n) {
    if (n.op != GHIP_OP_MUL_MAT || !n.src[0] || !n.src[1] || !n.dst) return false;
    const ghip_tensor *a = n.src[0], *b = n.src[1];
    // Q4_0 / Q5_0 / Q8_0: 1-8 F32 activation rows (the decode kernels' range)
    if (a->type == GHIP_TYPE_Q4_0 || a->type == GHIP_TYPE_Q5_0 || a->type == GHIP_TYPE_Q8_0)
        return b->type == GHIP_TYPE_F32 && b->ne[1] >= 1 && b->ne[1] <= 8 && b->ne[2] == 1 && b->ne[3] == 1 &&
               a->ne[2] == 1 && a->ne[3] == 1;
    if (a->type != GHIP_TYPE_Q4_K && a->type != GHIP_TYPE_Q5_K && a->type != GHIP_TYPE_Q6_K) return false;
    if (b->type != GHIP_TYPE_F32 || b->ne[1] < 1 || b->ne[2] != 1 || b->ne[3] != 1) return false;
    if (b->ne[1] > (a->type == GHIP_TYPE_Q6_K ? 1 : 8) && b->ne[1] < env_int("GHIP_GEMM_MIN_ROWS", 16))
        return false;
    if (b->ne[1] >= env_int("GHIP_GEMM_MIN_ROWS", 16))  // the prefill GEMM's range: Q4_K, 64-token tiles
        return a->type == GHIP_TYPE_Q4_K && gemm_bm() == 64 && b->ne[1] <= INT32_MAX &&
               std::string(getenv("GHIP_GEMM_KERNEL") ? getenv("GHIP_GEMM_KERNEL") : "") != "m128";
    if (a->ne[2] != 1 || a->ne[3] != 1) return false;
    return env_int("GHIP_GEMV_RB", 2) == 2 && env_int("GHIP_GEMV_NG", 2) == 2;
}
// node j joins the group nodes[i, j)
bool joins_group(const ghip_node *nodes, int i, int j) {
    const ghip_node &c = nodes[j], &h = nodes[i];
    if (!multi_candidate(c) || c.src[0]->type != h.src[0]->type || c.src[0]->ne[0] != h.src[0]->ne[0] ||
        !same_view(c.src[1], h.src[1]))
        return false;
    // Q4_K activations take the 4x8 values for the leading rows only when
    // N % 8 == 0 (compute.rs:5350-5398): one quantization per group
    if (c.src[0]->type == GHIP_TYPE_Q4_K && c.src[1]->ne[1] >= 4 && (c.src[0]->ne[1] % 8 == 0) != (h.src[0]->ne[1] % 8 == 0))
        return false;
    // the split-K and whole-K decode kernels sum differently: one kernel per group
    if (c.src[0]->type == GHIP_TYPE_Q4_K && sk_rows_ok(GHIP_TYPE_Q4_K, c.src[0]->ne[1]) != sk_rows_ok(GHIP_TYPE_Q4_K, h.src[0]->ne[1]))
        return false;
    // so do the matrix-core and VALU decode kernels, which a single op chooses
    // by its own row count at 4 activation rows (valu_q4k_small)
    if (c.src[0]->type == GHIP_TYPE_Q4_K && c.src[1]->ne[1] <= 4 && (c.src[0]->ne[1] < 8192) != (h.src[0]->ne[1] < 8192))
        return false;
    for (int k = i; k < j; k++) {
        const ghip_node &o = nodes[k];
        if (overlaps(o.dst, c.src[0]) || overlaps(o.dst, c.src[1]) || overlaps(c.dst, o.src[0]) ||
            overlaps(c.dst, o.src[1]) || overlaps(c.dst, o.dst))
            return false;
    }
    return true;
}

// Host mirror of GemmMulti in ghip_gemm.hip (kernel argument by value).
struct GemmMulti {
    const uint8_t *W[4];
    float *dst[4];
    int64_t ldd[4];
    int N[4];
    int t0[4];
    int n, total;
};

// 2..4 sibling Q4_K MUL_MATs with prefill-sized batches: one Q8_K
// quantization, one GEMM layout, one GEMM launch over all matrices' tiles
ghip_status mul_mat_multi_gemm(ghip_context *ctx, const ghip_node *nodes, int n, hipStream_t s) {
    std::lock_guard<std::mutex> lock(ctx->mu);
    MulMatPlan p[4];
    ghip_status st;
    for (int i = 0; i < n; i++) {
        if (!plan_mul_mat(ctx, nodes[i].src[0], nodes[i].src[1], nodes[i].dst, p[i], st)) return st;
        if (p[i].M != p[0].M || p[i].wtype != GHIP_TYPE_Q4_K || !use_gemm(p[i]) || p[i].act_pre)
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "graph_compute: internal: node not groupable");
    }
    if (!ctx->set_device()) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    st = ctx->begin(s);
    if (st != GHIP_STATUS_SUCCESS) return st;
    for (int i = 0; i < n; i++)
        ctx->allow(nodes[i].dst->data, win2d(p[i].M, (int64_t)nodes[i].dst->nb[1], p[i].N * 4, 1), "dst");
    const MulMatPlan &p0 = p[0];
    const int64_t Mpad = (p0.M + 127) / 128 * 128, K = p0.K, nbk = p0.K / 256;
    const size_t lay_bytes = (size_t)Mpad * K + (size_t)nbk * Mpad * 32 + (size_t)nbk * Mpad * 4;
    void *ws = nullptr;
    st = ctx->workspace(lay_bytes, s, &ws);
    if (st != GHIP_STATUS_SUCCESS) return st;
    int8_t *codes = (int8_t *)ws;
    uint16_t *bsT = (uint16_t *)(codes + Mpad * K);
    float *dT = (float *)(bsT + nbk * Mpad * 16);
    const ghip_tensor *bf = nodes[0].src[1];
    st = ctx->launch("ghip_gemm_act_q8K", dim3((unsigned)((p0.M * nbk + 3) / 4)), dim3(256), 0, s,
                     (const float *)bf->data, (int64_t)bf->nb[1] / 4, (int)p0.M, (int)Mpad, (int)nbk, (int)p0.n_mat,
                     codes, bsT, dT);
    if (st != GHIP_STATUS_SUCCESS) return st;
    GemmMulti g{};
    // the wide tiles when the group's tiles fill half a wave of workgroups
    int64_t wide_tiles = 0;
    for (int i = 0; i < n; i++) wide_tiles += gemm_tiles(kGemmW8, p0.M, p[i].N);
    const char *force = getenv("GHIP_GEMM_KERNEL");
    const bool wide = force && *force ? std::string(force) == "w8" : wide_tiles >= 128;
    const GemmKernel &gk = wide ? kGemmW8 : kGemmM64;
    int t = 0;
    for (int i = 0; i < n; i++) {
        g.W[i] = (const uint8_t *)nodes[i].src[0]->data;
        g.dst[i] = (float *)nodes[i].dst->data;
        g.ldd[i] = (int64_t)nodes[i].dst->nb[1] / 4;
        g.N[i] = (int)p[i].N;
        g.t0[i] = t;
        t += (int)gemm_tiles(gk, p0.M, p[i].N);
    }
    for (int i = n; i < 4; i++) {
        g.W[i] = g.W[0];
        g.dst[i] = g.dst[0];
        g.ldd[i] = g.ldd[0];
        g.N[i] = g.N[0];
        g.t0[i] = t;
    }
    g.n = n;
    g.total = t;
    return ctx->launch(gk.name_multi, dim3((unsigned)t), dim3(gk.threads), gk.smem, s, g,
                       (int64_t)p0.w_row_bytes, (int)nbk, (const int8_t *)codes, (const uint16_t *)bsT,
                       (const float *)dT, (int)p0.M, (int)Mpad);
}

// 2..4 sibling MUL_MATs (joins_group holds) as one multi-matrix GEMV launch
// pre_act: the group's activation rows already quantized to Q8_K (whole-K route)
ghip_status mul_mat_multi(ghip_context *ctx, const ghip_node *nodes, int n, hipStream_t s,
                          const uint8_t *pre_act = nullptr) {
    std::lock_guard<std::mutex> lock(ctx->mu);
    MulMatPlan p[4];
    ghip_status st;
    for (int i = 0; i < n; i++) {
        if (!plan_mul_mat(ctx, nodes[i].src[0], nodes[i].src[1], nodes[i].dst, p[i], st)) return st;
        if (p[i].M != p[0].M || p[i].M > 8 || !(gemv_v2(p[i]) || gemv_pair(p[i].wtype)) || p[i].act_pre)
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "graph_compute: internal: node not groupable");
    }
    if (!ctx->set_device()) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    st = ctx->begin(s);
    if (st != GHIP_STATUS_SUCCESS) return st;
    for (int i = 0; i < n; i++)
        ctx->allow(nodes[i].dst->data, win2d(p[i].M, (int64_t)nodes[i].dst->nb[1], p[i].N * 4, 1), "dst");
    const MulMatPlan &p0 = p[0];
    if (gemv_pair(p0.wtype)) {
        // Q8_0 rows once for the group, then 8 weight rows per workgroup
        const size_t act_bytes = ((size_t)(p0.M * p0.act_row_bytes) + 255) & ~(size_t)255;
        void *ws = nullptr;
        st = ctx->workspace(act_bytes, s, &ws);
        if (st != GHIP_STATUS_SUCCESS) return st;
        st = quantize_act(ctx, p0, nodes[0].src[1], ws, s);
        if (st != GHIP_STATUS_SUCCESS) return st;
        const int wk = (int)(((p0.nb + 1) / 2 + 63) / 64);
        if (wk > 8) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: ne00 = %lld too large for the decode kernel", (long long)p0.K);
        GemvMulti g{};
        int wgs = 0;
        for (int i = 0; i < 4; i++) {
            const int j = i < n ? i : 0;
            g.W[i] = (const uint8_t *)nodes[j].src[0]->data;
            g.dst[i] = (float *)nodes[j].dst->data;
            g.ldd[i] = (int64_t)nodes[j].dst->nb[1] / 4;
            g.rows[i] = i < n ? (int)p[i].N : 0;
            g.wg0[i] = wgs;
            if (i < n) wgs += (int)((p[i].N + 7) / 8);
        }
        g.n = n;
        const int nc = (int)p0.M;
        const int NC = nc == 1 ? 1 : nc == 2 ? 2 : nc <= 4 ? 4 : 8;
        return ctx->launch(std::string(gemv_base(p0.wtype)) + "_c" + std::to_string(NC) + "_multi", dim3((unsigned)wgs),
                           dim3(64 * wk), 0, s, g, (int64_t)p0.w_row_bytes, (int)p0.nb, (const uint8_t *)ws,
                           (int64_t)p0.act_row_bytes, nc);
    }
    if (use_sq(p0)) {
        // the activation rows quantized once (here or before the graph's first
        // node), then the whole-K kernel over all members
        void *ws = (void *)pre_act;
        if (!ws) {
            const size_t act_bytes = ((size_t)(p0.M * p0.act_row_bytes) + 255) & ~(size_t)255;
            st = ctx->workspace(act_bytes, s, &ws);
            if (st != GHIP_STATUS_SUCCESS) return st;
            st = quantize_act(ctx, p0, nodes[0].src[1], ws, s);
            if (st != GHIP_STATUS_SUCCESS) return st;
        }
        SkLaunch g{};
        g.n = n;
        for (int i = 0; i < n; i++) {
            g.m[i].W = (const uint8_t *)nodes[i].src[0]->data;
            g.m[i].dst = (float *)nodes[i].dst->data;
            g.m[i].ldd = (int64_t)nodes[i].dst->nb[1] / 4;
            g.m[i].rows = (int)p[i].N;
        }
        return launch_sq(ctx, p0, g, (const uint8_t *)ws, p0.act_row_bytes, nullptr, s);
    }
    if (use_sk(p0)) {
        // split-K decode over all members; partials of member i after member i-1's
        size_t off[4] = {0, 0, 0, 0}, total = 0;
        for (int i = 0; i < n; i++) {
            off[i] = total;
            total += sk_part_bytes(p[i]);
        }
        void *ws = nullptr;
        if (total) {
            st = ctx->workspace(total, s, &ws);
            if (st != GHIP_STATUS_SUCCESS) return st;
        }
        SkLaunch g{};
        g.n = n;
        for (int i = 0; i < n; i++) {
            g.m[i].W = (const uint8_t *)nodes[i].src[0]->data;
            g.m[i].dst = (float *)nodes[i].dst->data;
            g.m[i].ldd = (int64_t)nodes[i].dst->nb[1] / 4;
            g.m[i].part = ws ? (float *)((uint8_t *)ws + off[i]) : nullptr;
            g.m[i].rows = (int)p[i].N;
        }
        return launch_sk(ctx, p0, g, nodes[0].src[1], nullptr, s);
    }
    if (use_skinny(p0)) {
        // Q4_K at 4..15 rows: the activation rows quantized once, then the
        // matrix-core decode kernel over all members
        int NC, RT, KS;
        skinny_shape(p0.M, NC, RT, KS);
        RT = 2, KS = 4;  // the single-op default (grouped kernels exist for it)
        const size_t shmem = skinny_lds(NC, p0.K, p0.nb);
        if (shmem > 160 * 1024) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: decode LDS image too large");
        const size_t act_bytes = ((size_t)(p0.M * p0.act_row_bytes) + 255) & ~(size_t)255;
        void *ws = nullptr;
        st = ctx->workspace(act_bytes, s, &ws);
        if (st != GHIP_STATUS_SUCCESS) return st;
        st = quantize_act(ctx, p0, nodes[0].src[1], ws, s);
        if (st != GHIP_STATUS_SUCCESS) return st;
        GemvMulti g{};
        int wg = 0;
        for (int i = 0; i < 4; i++) {
            const int j = i < n ? i : 0;
            g.W[i] = (const uint8_t *)nodes[j].src[0]->data;
            g.dst[i] = (float *)nodes[j].dst->data;
            g.ldd[i] = (int64_t)nodes[j].dst->nb[1] / 4;
            g.rows[i] = i < n ? (int)p[i].N : 0;
            g.wg0[i] = wg;
            if (i < n) wg += (int)((p[i].N + 16 * RT - 1) / (16 * RT));
        }
        g.n = n;
        const int n_mat = (int)std::max<int64_t>(0, std::min<int64_t>(p0.M, p0.n_mat));
        const std::string name = "ghip_mma_q4_K_c" + std::to_string(NC) + "_r" + std::to_string(RT) + "k" +
                                 std::to_string(KS) + "_multi";
        return ctx->launch(name, dim3((unsigned)wg), dim3(512), shmem, s, g, (int64_t)p0.w_row_bytes, (int)p0.nb,
                           (const uint8_t *)ws, (int64_t)p0.act_row_bytes, (int)p0.M, n_mat);
    }
    const int waves_k = (int)((p0.nb + 15) / 16);
    if (waves_k > 8) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: ne00 = %lld too large for the decode kernel", (long long)p0.K);
    // 8 row teams per workgroup: measured on q/k/v (4096 + 1024 + 1024 rows)
    // 6.8 -> 5.9 us at batch 1 and 9.1 -> 7.8 us at batch 2 against 4 teams;
    // gate/up (2 x 14336) within 2 % either way
    int64_t rows_total = 0;
    for (int i = 0; i < n; i++) rows_total += p[i].N;
    int rb, ng, ns = 2, teams = std::max(1, std::min(8 / waves_k, env_int("GHIP_GEMV_TEAMS", 8)));
    gemv_groups(p0.wtype, p0.M, rows_total, rb, ng);
    if (p0.wtype == GHIP_TYPE_Q5_K) rb = ng = 2;
    if (p0.wtype == GHIP_TYPE_Q4_K && p0.M <= 4 && waves_k == 1) {
        int t;
        rb = 1;
        gemv_q4k_one_row(rows_total, t, ng, ns);
        if (p0.M > 2) t = 8, ng = 2, ns = 2, rb = rows_total < 8192 ? 1 : 2;  // as in the single-matrix rule
        teams = std::max(1, std::min(8, env_int("GHIP_GEMV_TEAMS", t)));
        ng = env_int("GHIP_GEMV_NG", ng);
        ns = env_int("GHIP_GEMV_NS", ns);
    }
    const int rows_per_wg = rb * ng * teams;
    GemvMulti g{};
    int wg = 0;
    for (int i = 0; i < n; i++) {
        g.W[i] = (const uint8_t *)nodes[i].src[0]->data;
        g.dst[i] = (float *)nodes[i].dst->data;
        g.ldd[i] = (int64_t)nodes[i].dst->nb[1] / 4;
        g.rows[i] = (int)p[i].N;
        g.wg0[i] = wg;
        wg += (int)((p[i].N + rows_per_wg - 1) / rows_per_wg);
    }
    for (int i = n; i < 4; i++) {
        g.W[i] = g.W[0];
        g.dst[i] = g.dst[0];
        g.ldd[i] = g.ldd[0];
        g.rows[i] = 0;
        g.wg0[i] = wg;
    }
    g.n = n;
    const int nc = (int)p0.M;
    const int NC = nc == 1 ? 1 : nc == 2 ? 2 : nc <= 4 ? 4 : 8;
    const size_t shmem = (size_t)NC * p0.K + (size_t)NC * p0.nb * 4 + (size_t)NC * p0.nb * 16 * 4 +
                         (size_t)rows_per_wg * waves_k * NC * sizeof(float);
    if (shmem > 160 * 1024) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: decode LDS image too large");
    const std::string name = std::string(gemv_base(p0.wtype)) + (p0.wtype == GHIP_TYPE_Q6_K ? "_v2" : "") + "_f_c" +
                             std::to_string(NC) + "_r" + std::to_string(rb) + "x" + std::to_string(ng) +
                             (ns != 2 ? "s" + std::to_string(ns) : std::string()) + "_multi";
    const int n_mat = p0.wtype == GHIP_TYPE_Q5_K ? (p0.M >= 8 ? -1 : 0)  // as in run_gemv
                                                 : (int)std::max<int64_t>(0, std::min<int64_t>(nc, p0.n_mat));
    return ctx->launch(name, dim3((unsigned)wg), dim3(64 * waves_k * teams), shmem, s, g, (int64_t)p0.w_row_bytes,
                       (int)p0.nb, (const uint8_t *)nodes[0].src[1]->data, (int64_t)nodes[0].src[1]->nb[1], nc,
                       n_mat);
}

}  // namespace

extern "C" {

ghip_status ghip_mul_mat_id(ghip_context *ctx, const ghip_tensor *as, const ghip_tensor *b, const ghip_tensor *ids,
                            const ghip_tensor *dst, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    if (!dst) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat_id: null dst");
    return mul_mat_id_impl(ctx, as, b, ids, dst, nullptr, stream);
}

ghip_status ghip_mul_mat_id_subsums(ghip_context *ctx, const ghip_tensor *as, const ghip_tensor *b,
                                    const ghip_tensor *ids, int32_t *subsums, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    if (!subsums) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat_id_subsums: null output");
    return mul_mat_id_impl(ctx, as, b, ids, nullptr, subsums, stream);
}

// one sequence (q, k, v, mask plane and dst of one i3)
static ghip_status fa_sequence(ghip_context *ctx, const ghip_tensor *q, const ghip_tensor *k, const ghip_tensor *v,
                        const ghip_tensor *mask, const ghip_tensor *sinks, const ghip_tensor *dst, void *stream) {
    std::lock_guard<std::mutex> lock(ctx->mu);
    ghip_status st;
    if (!plan_fa(ctx, q, k, v, mask, sinks, dst, st)) return st;
    const int D = (int)k->ne[0], T = (int)q->ne[1], H = (int)q->ne[2], S = (int)k->ne[1], H_kv = (int)k->ne[2];
    if (T == 0 || H == 0) return GHIP_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;
    if (!ctx->set_device()) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    st = ctx->begin(s);
    if (st != GHIP_STATUS_SUCCESS) return st;
    const FaLayout L = fa_layout(D, T, H, S, H_kv, mask ? (int)mask->ne[2] : 0);
    const int G = L.G, QS = L.QS, qtiles = L.qtiles;
    int nsplit = L.nsplit, chunk = L.chunk;
    void *ws = nullptr;
    if (L.ws_bytes) {
        st = ctx->workspace(L.ws_bytes, s, &ws);
        if (st != GHIP_STATUS_SUCCESS) return st;
    }
    FaParams p;
    p.q = (const float *)q->data;
    p.q_nb1 = (int64_t)q->nb[1] / 4;
    p.q_nb2 = (int64_t)q->nb[2] / 4;
    p.k = (const uint16_t *)k->data;
    p.v = (const uint16_t *)v->data;
    p.k_nb1 = (int64_t)k->nb[1] / 2;
    p.k_nb2 = (int64_t)k->nb[2] / 2;
    p.v_nb1 = (int64_t)v->nb[1] / 2;
    p.v_nb2 = (int64_t)v->nb[2] / 2;
    p.mask = mask ? (const uint16_t *)mask->data : nullptr;
    p.mask_nb1 = mask ? (int64_t)mask->nb[1] / 2 : 0;
    p.mask_nb2 = mask ? (int64_t)mask->nb[2] / 2 : 0;
    p.mask_ne2 = mask ? (int)mask->ne[2] : 1;
    p.dst = (float *)dst->data;
    p.part = (float *)ws;
    p.T = T;
    p.S = S;
    p.H = H;
    p.H_kv = H_kv;
    p.nsplit = nsplit;
    p.chunk = chunk;
    const float scale = f32_param(dst, 0), max_bias = f32_param(dst, 1), softcap = f32_param(dst, 2);
    // flash_attn.rs:391-413: scale is pre-divided by the softcap; ALiBi slopes
    p.scale = softcap != 0.0f ? scale / softcap : scale;
    p.softcap = softcap;
    p.n_head_log2 = 1 << (int)std::floor(std::log2((double)H));
    p.m0 = max_bias > 0.0f ? powf(2.0f, -max_bias / (float)p.n_head_log2) : 1.0f;
    p.m1 = max_bias > 0.0f ? powf(2.0f, -(max_bias / 2.0f) / (float)p.n_head_log2) : 1.0f;
    p.sinks = sinks ? (const float *)sinks->data : nullptr;
    p.DK = D;
    p.DV = (int)v->ne[0];
    p.k_f32 = k->type == GHIP_TYPE_F32;
    p.v_f32 = v->type == GHIP_TYPE_F32;
    p.mflags = nullptr;
    p.nqb = L.nqb;
    p.ntile = L.ntile;
    p.direct = 0;
    // shapes the tuned kernels do not take (F32 K or V, DK != DV, head sizes
    // other than 64 / 128, H / H_kv > 8) run the general row walk: with the
    // f16 accumulator where the reference's route is the row walk over an F16
    // V, fp32 otherwise
    // (the split-KV decode kernel reads one mask value per key for all G
    // heads of a KV head, so per-head mask planes take the row walk too)
    const bool per_head_mask = mask && mask->ne[2] > 1;
    const bool tuned = !p.k_f32 && !p.v_f32 && p.DK == p.DV && (D == 64 || D == 128) && G <= 8 &&
                       !(per_head_mask && T == 1 && S >= 512);
    if (!tuned) {
        const bool row_walk = !(T == 1 && S >= 512) && T < 64;
        return ctx->launch(row_walk && !p.v_f32 ? "ghip_fa_rowgen_f16acc" : "ghip_fa_rowgen",
                           dim3((unsigned)((T * H + 3) / 4)), dim3(256), 0, s, p);
    }
    // flash_attn.rs:371-386 routes: single-row decode over >= 512 keys splits the
    // KV range, >= 64 query rows take the tiled kernel (fp32 accumulators) --
    // both run on the MFMA kernel below.  Fewer rows take the one-chunk walk
    // with its f16 accumulator, reproduced by the row-sequential kernel.
    if (!(T == 1 && S >= 512) && T < 64 && !env_int("GHIP_FA_FORCE_MFMA", 0)) {
        const char *rs = D == 128 ? "ghip_fa_rowseq_d128" : "ghip_fa_rowseq_d64";
        return ctx->launch(rs, dim3((unsigned)((T * H + 3) / 4)), dim3(256), 0, s, p);
    }
    if (T == 1) {
        // single-query split-KV route: the bandwidth-bound vector kernel
        const int ns = nsplit;
        const char *dec = D == 128 ? "ghip_fa_decode_d128" : "ghip_fa_decode_d64";
        st = ctx->launch(dec, dim3(H_kv, ns), dim3(256), 0, s, p);
        if (st != GHIP_STATUS_SUCCESS) return st;
        if (ns <= 64)
            return ctx->launch("ghip_fa_merge_rows4", dim3((unsigned)H), dim3(256), 0, s, (const float *)ws, p.sinks,
                               (float *)dst->data, H, H, ns, D);
        return ctx->launch("ghip_fa_merge", dim3((unsigned)H), dim3(256), 0, s, (const float *)ws, p.sinks,
                           (float *)dst->data, 1, H, ns, D);
    }
    const char *fwd = softcap != 0.0f ? (D == 128 ? "ghip_fa_fwd_sc_d128" : "ghip_fa_fwd_sc_d64")
                                      : (D == 128 ? "ghip_fa_fwd_d128" : "ghip_fa_fwd_d64");
    if (mask && L.ws_bytes > L.flags_off) {
        // classes of the mask's (32-query, 64-key) tiles: the forward kernel
        // skips the loads of all-zero tiles and the work of all -inf ones
        // (a causal mask is mostly the former; loading it cost 20 of 154 us
        // at T = 512, S = 8192)
        uint8_t *fl = (uint8_t *)ws + L.flags_off;
        const int64_t nfl = (int64_t)mask->ne[2] * L.nqb * L.ntile;
        ctx->expect(fl, (size_t)nfl, "mask tile classes");
        st = ctx->launch("ghip_fa_mask_scan", dim3((unsigned)((nfl + 3) / 4)), dim3(256), 0, s, p.mask, p.mask_nb1,
                         p.mask_nb2, (int)mask->ne[2], T, S, L.nqb, L.ntile, fl);
        if (st != GHIP_STATUS_SUCCESS) return st;
        p.mflags = fl;
    }
    // one KV slice (long prefills: every query tile and KV head already fills
    // the GPU): the forward kernel writes the normalized rows, no merge
    p.direct = nsplit == 1 && env_int("GHIP_FA_DIRECT", 1) != 0;
    st = ctx->launch(fwd, dim3((unsigned)(qtiles * H_kv * nsplit)), dim3(64 * G * QS), 0, s, p);
    if (st != GHIP_STATUS_SUCCESS || p.direct) return st;
    const float *sk = sinks ? (const float *)sinks->data : nullptr;
    if (nsplit <= 64)
        return ctx->launch(nsplit <= 4 && env_int("GHIP_FA_MERGE_P4", 1) ? "ghip_fa_merge_rows_p4" : "ghip_fa_merge_rows",
                           dim3((unsigned)((T * H + 3) / 4)), dim3(256), 0, s,
                           (const float *)ws, sk, (float *)dst->data, T * H, H, nsplit, D);
    return ctx->launch("ghip_fa_merge", dim3((unsigned)(T * H)), dim3(256), 0, s, (const float *)ws, sk,
                       (float *)dst->data, T, H, nsplit, D);
}

// FLASH_ATTN_EXT over sequences (dim 3, flash_attn.rs:298): sequence i3 reads
// q, k and v plane i3 and mask plane i3 % mask_ne3 and writes dst plane i3
ghip_status ghip_flash_attn_ext(ghip_context *ctx, const ghip_tensor *q, const ghip_tensor *k, const ghip_tensor *v,
                                const ghip_tensor *mask, const ghip_tensor *sinks, const ghip_tensor *dst,
                                void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    if (!q || !k || !v || !dst || q->ne[3] == 1)
        return fa_sequence(ctx, q, k, v, mask, sinks, dst, stream);
    {
        std::lock_guard<std::mutex> lock(ctx->mu);
        ghip_status st;
        if (!plan_fa(ctx, q, k, v, mask, sinks, dst, st)) return st;
    }
    for (int64_t i3 = 0; i3 < q->ne[3]; i3++) {
        ghip_tensor q2 = *q, k2 = *k, v2 = *v, d2 = *dst, m2;
        q2.data = (uint8_t *)q->data + i3 * q->nb[3];
        k2.data = (uint8_t *)k->data + i3 * k->nb[3];
        v2.data = (uint8_t *)v->data + i3 * v->nb[3];
        d2.data = (uint8_t *)dst->data + i3 * dst->nb[3];
        q2.ne[3] = k2.ne[3] = v2.ne[3] = d2.ne[3] = 1;
        if (mask) {
            m2 = *mask;
            m2.data = (uint8_t *)mask->data + (i3 % mask->ne[3]) * mask->nb[3];
            m2.ne[3] = 1;
        }
        const ghip_status st = fa_sequence(ctx, &q2, &k2, &v2, mask ? &m2 : nullptr, sinks, &d2, stream);
        if (st != GHIP_STATUS_SUCCESS) return st;
    }
    return GHIP_STATUS_SUCCESS;
}


ghip_status ghip_init(int device, ghip_context **out) {
    if (!out) return GHIP_STATUS_BACKEND_ERROR;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) {
        (void)hipGetLastError();
        return GHIP_STATUS_BACKEND_ERROR;
    }
    if (hipSetDevice(device) != hipSuccess) return GHIP_STATUS_BACKEND_ERROR;
    ghip_context *ctx = new ghip_context();
    ctx->device = device;
    ctx->check_stores = env_int("GHIP_CHECK_STORES", 0) != 0;
    const char *why = "";
    if (ghip_noalloc_setup(device, &why) != GHIP_STATUS_SUCCESS ||
        hipEventCreateWithFlags(&ctx->order_ev, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        fprintf(stderr, "ghip: init on device %d failed: %s\n", device, *why ? why : "hipEventCreate failed");
        delete ctx;
        return GHIP_STATUS_BACKEND_ERROR;
    }
    const std::string dir = library_dir();
    for (const char *m : kModules) {
        hipModule_t mod;
        const std::string path = dir + "/" + m;
        if (hipModuleLoad(&mod, path.c_str()) != hipSuccess) {
            fprintf(stderr, "ghip: cannot load code object %s\n", path.c_str());
            (void)hipGetLastError();
            for (hipModule_t x : ctx->modules) hipModuleUnload(x);
            delete ctx;
            return GHIP_STATUS_BACKEND_ERROR;
        }
        ctx->modules.push_back(mod);
    }
    *out = ctx;
    return GHIP_STATUS_SUCCESS;
}

ghip_status ghip_init_dry_run(ghip_context **out) {
    if (!out) return GHIP_STATUS_BACKEND_ERROR;
    ghip_context *ctx = new ghip_context();
    ctx->dry_run = true;
    ctx->check_stores = true;
    *out = ctx;
    return GHIP_STATUS_SUCCESS;
}

void ghip_free(ghip_context *ctx) {
    if (!ctx) return;
    if (ctx->dry_run) {
        delete ctx;
        return;
    }
    hipSetDevice(ctx->device);
    hipDeviceSynchronize();
    if (ctx->ws) hipFree(ctx->ws);
    for (void *p : ctx->retired) hipFree(p);
    for (auto &kv : ctx->wcache) hipFree(kv.second.p);
    for (int b = 0; b < 2; b++) {
        if (ctx->stage[b]) hipHostFree(ctx->stage[b]);
        if (ctx->stage_ev[b]) hipEventDestroy(ctx->stage_ev[b]);
    }
    if (ctx->order_ev) hipEventDestroy(ctx->order_ev);
    for (hipModule_t m : ctx->modules) hipModuleUnload(m);
    delete ctx;
}

static bool repack_enabled() {
    const char *v = getenv("LLAMA_RUST_REPACK");
    return !v || !(strcmp(v, "0") == 0 || strcasecmp(v, "false") == 0);
}

static size_t repack_budget() {
    const char *v = getenv("LLAMA_RUST_REPACK_MAX_MB");
    const long long mb = v && *v ? atoll(v) : 16384;
    return (size_t)std::max(0LL, mb) << 20;
}

ghip_status ghip_weight_register(ghip_context *ctx, const ghip_tensor *w, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (!w || !w->data) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_register: null weight");
    if (w->ne[0] <= 0 || w->ne[1] <= 0 || w->ne[2] <= 0 || w->ne[3] != 1)
        return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_register: empty or 4-D weight");
    const bool q6k = w->type == GHIP_TYPE_Q6_K, mx = w->type == GHIP_TYPE_MXFP4, q8 = gemm_q8_family(w->type);
    if ((q6k || q8) && w->ne[2] != 1)
        return ctx->fail(GHIP_STATUS_BACKEND_ERROR,
                         "weight_register: Q6_K / Q4_0 / Q5_0 / Q8_0 / IQ4_NL / IQ4_XS / Q1_0 / Q2_0 weights are 2-D");
    // every other type is read in its GGUF layout: nothing to build
    if (!(q6k || mx || q8) || !repack_enabled()) return GHIP_STATUS_SUCCESS;
    size_t bytes;
    int64_t nbk = 0, nrb = 0, ngp = 0;
    Q8Layout QL{};
    if (q8) {
        const TypeInfo ti = type_info(w->type);
        if (w->ne[0] % ti.blck || w->nb[0] != (uint64_t)ti.bytes || w->nb[1] < (uint64_t)(w->ne[0] / ti.blck * ti.bytes))
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_register: bad block geometry");
        if (w->ne[1] > INT32_MAX) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_register: dimension too large");
        QL = q8_layout(1, w->ne[1], w->ne[0]);
        bytes = QL.w_b + QL.dw_b + q8_extra_b(w->type, QL);
    } else if (q6k) {
        if (w->ne[0] % 256 || w->nb[0] != 210 || w->nb[1] < (uint64_t)(w->ne[0] / 256 * 210))
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_register: bad Q6_K geometry");
        if (w->ne[1] > INT32_MAX || w->ne[0] / 256 > INT32_MAX)
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_register: dimension too large");
        nbk = w->ne[0] / 256;
        bytes = (size_t)w->ne[1] * (size_t)nbk * kQ6R;
    } else {
        if (w->ne[0] % 32 || w->nb[0] != 17 || w->nb[1] < (uint64_t)(w->ne[0] / 32 * 17) ||
            (w->ne[2] > 1 && w->nb[2] < w->nb[1] * (uint64_t)w->ne[1]))
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_register: bad MXFP4 geometry");
        if (w->ne[1] > INT32_MAX || w->ne[2] > INT32_MAX)
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_register: dimension too large");
        nrb = (w->ne[1] + kMoeRows - 1) / kMoeRows;
        ngp = (w->ne[0] / 32 + kMoeGroup - 1) / kMoeGroup;
        bytes = (size_t)w->ne[2] * (size_t)nrb * (size_t)ngp * kMoeWindowRun;
    }
    const ghip_context::WeightKey key = ghip_context::key_of(w);
    if (ctx->wcache.count(key)) return GHIP_STATUS_SUCCESS;
    if (ctx->wcache_bytes + bytes > repack_budget()) return GHIP_STATUS_SUCCESS;  // not kept: calls repack per call
    hipStream_t s = (hipStream_t)stream;
    if (ghip_context::capturing(s))
        return ctx->fail(GHIP_STATUS_ALLOC_FAILED, "weight_register allocates: not while the stream is captured");
    if (!ctx->set_device()) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    ghip_status st = ctx->begin(s);
    if (st != GHIP_STATUS_SUCCESS) return st;
    void *rep = nullptr;
    if (hipMalloc(&rep, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return ctx->fail(GHIP_STATUS_OUT_OF_MEMORY, "weight_register: hipMalloc(%zu) failed", bytes);
    }
    if (q8) {
        st = q8w_repack(ctx, w->type, w->data, (int64_t)w->nb[1], w->ne[1], w->ne[0] / type_info(w->type).blck, QL, (int8_t *)rep,
                        (float *)((uint8_t *)rep + QL.w_b), s);
    } else if (q6k) {
        st = q6k_repack(ctx, w->data, (int64_t)w->nb[1], w->ne[1], nbk, (uint8_t *)rep, s);
    } else {
        const int64_t chunks = (int64_t)(bytes / 16);
        st = ctx->launch("ghip_mxfp4_repack", dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, s,
                         (const uint8_t *)w->data, (int64_t)w->nb[1], (int64_t)(w->ne[2] > 1 ? w->nb[2] : 0),
                         (int)w->ne[1], (int)(w->ne[0] / 32), (int)w->ne[2], (int)nrb, (int)ngp, (uint8_t *)rep);
    }
    if (st != GHIP_STATUS_SUCCESS) {
        hipFree(rep);
        return st;
    }
    ctx->wcache.emplace(key, ghip_context::WeightCopy{rep, bytes});
    ctx->wcache_bytes += bytes;
    ctx->wcache_built++;
    return GHIP_STATUS_SUCCESS;
}

ghip_status ghip_weight_unregister(ghip_context *ctx, const ghip_tensor *w) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (!w) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_unregister: null weight");
    auto it = ctx->wcache.find(ghip_context::key_of(w));
    if (it == ctx->wcache.end()) return GHIP_STATUS_SUCCESS;
    if (hipSetDevice(ctx->device) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        (void)hipGetLastError();
        return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "weight_unregister: device synchronize failed");
    }
    hipFree(it->second.p);
    ctx->wcache_bytes -= it->second.bytes;
    ctx->wcache.erase(it);
    return GHIP_STATUS_SUCCESS;
}

ghip_status ghip_weight_cache_stats(ghip_context *ctx, size_t *n_weights, size_t *bytes, size_t *built) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (n_weights) *n_weights = ctx->wcache.size();
    if (bytes) *bytes = ctx->wcache_bytes;
    if (built) *built = ctx->wcache_built;
    return GHIP_STATUS_SUCCESS;
}

const char *ghip_last_error(const ghip_context *ctx) { return ctx ? ctx->err.c_str() : "null context"; }

ghip_status ghip_synchronize(ghip_context *ctx, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    const hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipStreamSynchronize: %s", hipGetErrorString(e));
    return GHIP_STATUS_SUCCESS;
}

int ghip_supports_op(int op, const ghip_tensor *dst, const ghip_tensor *const *srcs, int n_srcs) {
    if (op == GHIP_OP_MUL_MAT) {
        if (n_srcs < 2 || !srcs[0] || !srcs[1]) return 0;
        ghip_context tmp;
        MulMatPlan p;
        ghip_status st;
        return plan_mul_mat(&tmp, srcs[0], srcs[1], dst, p, st) ? 1 : 0;
    }
    if (op == GHIP_OP_MUL_MAT_ID) {
        if (n_srcs < 3 || !srcs[0] || !srcs[1] || !srcs[2]) return 0;
        ghip_context tmp;
        MoePlan p;
        ghip_status st;
        return plan_moe(&tmp, srcs[0], srcs[1], srcs[2], dst, p, st) ? 1 : 0;
    }
    if (op == GHIP_OP_FLASH_ATTN_EXT) {
        if (n_srcs < 3 || !dst) return 0;
        ghip_context tmp;
        ghip_status st;
        return plan_fa(&tmp, srcs[0], srcs[1], srcs[2], n_srcs > 3 ? srcs[3] : nullptr,
                       n_srcs > 4 ? srcs[4] : nullptr, dst, st) ? 1 : 0;
    }
    return 0;
}

ghip_status ghip_mul_mat(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1, const ghip_tensor *dst,
                         void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    if (!dst) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: null dst");
    return mul_mat_impl(ctx, src0, src1, dst, nullptr, nullptr, stream);
}

}  // extern "C"

ghip_status ghip_mul_mat_fixed_scratch(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1,
                                       const ghip_tensor *dst, void *scratch, size_t bytes, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    if (!dst) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: null dst");
    return mul_mat_impl(ctx, src0, src1, dst, nullptr, nullptr, stream, scratch, bytes);
}
int ghip_context_device(const ghip_context *ctx) { return ctx ? ctx->device : -1; }

ghip_status ghip_context_upload(ghip_context *ctx, void *dst, const void *src, size_t n, void *stream) {
    constexpr size_t kStage = 32u << 20;
    std::lock_guard<std::mutex> lock(ctx->mu);
    hipStream_t s = (hipStream_t)stream;
    if (ghip_context::capturing(s)) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "gguf_upload: stream is being captured");
    if (!ctx->set_device()) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    for (int b = 0; b < 2; b++) {
        if (!ctx->stage[b] && (hipHostMalloc(&ctx->stage[b], kStage, hipHostMallocDefault) != hipSuccess ||
                               hipEventCreateWithFlags(&ctx->stage_ev[b], hipEventDisableTiming) != hipSuccess)) {
            (void)hipGetLastError();
            return ctx->fail(GHIP_STATUS_OUT_OF_MEMORY, "gguf_upload: pinned staging allocation failed");
        }
    }
    ghip_status st = ctx->begin(s);
    if (st != GHIP_STATUS_SUCCESS) return st;
    bool used[2] = {false, false};
    for (size_t off = 0, k = 0; off < n; off += kStage, k++) {
        const int b = (int)(k & 1);
        const size_t len = std::min(kStage, n - off);
        // (a staging buffer whose last copy did not finish must not be
        // refilled, and the tensor would be left partly uploaded)
        if (used[b] && hipEventSynchronize(ctx->stage_ev[b]) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipStreamSynchronize(s);
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "gguf_upload: staging wait failed");
        }
        memcpy(ctx->stage[b], (const uint8_t *)src + off, len);
        if (hipMemcpyAsync((uint8_t *)dst + off, ctx->stage[b], len, hipMemcpyHostToDevice, s) != hipSuccess ||
            hipEventRecord(ctx->stage_ev[b], s) != hipSuccess) {
            (void)hipGetLastError();
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "gguf_upload: host-to-device copy failed");
        }
        used[b] = true;
    }
    if (hipStreamSynchronize(s) != hipSuccess) {
        (void)hipGetLastError();
        return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "gguf_upload: copy did not complete");
    }
    return GHIP_STATUS_SUCCESS;
}
ghip_status ghip_context_fail(ghip_context *ctx, ghip_status st, const char *msg) { return ctx->fail(st, "%s", msg); }

extern "C" {

ghip_status ghip_mul_mat_subsums(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1,
                                 int32_t *subsums, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    if (!subsums) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat_subsums: null output");
    return mul_mat_impl(ctx, src0, src1, nullptr, subsums, nullptr, stream);
}

ghip_status ghip_mul_mat_act(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1, void *out,
                             void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    if (!out) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat_act: null output");
    return mul_mat_impl(ctx, src0, src1, nullptr, nullptr, out, stream);
}

// Host mirror of Q8KSegs in ghip_quant.hip.
struct Q8KSegs {
    const float *x[8];
    int64_t x_stride[8];
    uint8_t *y[8];
    int64_t y_stride[8];
    int64_t nb[8];
    int64_t n_mat[8];
    int64_t w0[9];
    int n;
};

// ghip_graph_compute's inputs are ready when it is called: a group on the
// whole-K decode route whose f32 activation rows no earlier node writes has
// them quantized before the first node, all such groups in one launch
// (ghip_quantize_q8_K_segs) instead of one quantize launch each.  The Q8_K
// rows stay at the start of the workspace (ctx->hold) until the call ends;
// group gi reads them through pre[gi] (pre_view[gi]: a Q8_K view for a single
// node).  Each group keeps its own quantization (its n_mat rule); groups with
// the same rows and rule share them.  GHIP_GRAPH_PREQUANT=0 turns this off;
// so does a workspace given with ghip_set_workspace.
ghip_status prequantize(ghip_context *ctx, const ghip_node *nodes, const std::vector<std::pair<int, int>> &groups,
                        std::vector<const uint8_t *> &pre, std::vector<ghip_tensor> &pre_view, hipStream_t s) {
    // (a caller's workspace is sized per node, by ghip_workspace_size: the
    // held rows would not fit beside the largest node's)
    if (env_int("GHIP_GRAPH_PREQUANT", 1) == 0 || env_int("GHIP_GRAPH_FUSE", 1) == 0 || ctx->user_ws || ctx->call_ws)
        return GHIP_STATUS_SUCCESS;
    struct Seg {
        const ghip_tensor *x;
        MulMatPlan p;
        size_t off;
    };
    std::vector<Seg> segs;
    std::vector<int> seg_of(groups.size(), -1);
    size_t total = 0;
    for (size_t gi = 0; gi < groups.size(); gi++) {
        const ghip_node &nd = nodes[groups[gi].first];
        if (nd.op != GHIP_OP_MUL_MAT || !nd.src[0] || !nd.src[1] || !nd.dst) continue;
        const ghip_tensor *x = nd.src[1];
        if (x->type != GHIP_TYPE_F32 || x->ne[2] != 1 || x->ne[3] != 1) continue;
        MulMatPlan p;
        ghip_status st;
        {
            std::lock_guard<std::mutex> lock(ctx->mu);
            if (!plan_mul_mat(ctx, nd.src[0], x, nd.dst, p, st)) {
                ctx->err.clear();
                continue;  // the node itself reports it
            }
        }
        if (!use_sq(p) || p.act_pre || p.M == 0 || p.N == 0) continue;
        bool ready = true;
        for (int k = 0; k < groups[gi].first && ready; k++) ready = !overlaps(nodes[k].dst, x);
        if (!ready) continue;
        int found = -1;
        for (size_t j = 0; j < segs.size() && found < 0; j++)
            if (same_view(segs[j].x, x) && segs[j].p.n_mat == p.n_mat && segs[j].p.K == p.K) found = (int)j;
        if (found < 0) {
            if (segs.size() == 8) continue;
            segs.push_back({x, p, total});
            total += ((size_t)(p.M * p.act_row_bytes) + 255) & ~(size_t)255;
            found = (int)segs.size() - 1;
        }
        seg_of[gi] = found;
    }
    if (segs.size() < 2) return GHIP_STATUS_SUCCESS;  // nothing to save over the groups' own launches
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (!ctx->set_device()) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    ghip_status st = ctx->begin(s);
    if (st != GHIP_STATUS_SUCCESS) return st;
    void *ws = nullptr;
    st = ctx->workspace(total, s, &ws);
    if (st != GHIP_STATUS_SUCCESS) return st;
    Q8KSegs g{};
    int64_t waves = 0;
    for (size_t j = 0; j < segs.size(); j++) {
        const MulMatPlan &p = segs[j].p;
        uint8_t *y = (uint8_t *)ws + segs[j].off;
        ctx->expect(y, (size_t)(p.M * p.act_row_bytes), "quantized activations");
        g.x[j] = (const float *)segs[j].x->data;
        g.x_stride[j] = (int64_t)segs[j].x->nb[1] / 4;
        g.y[j] = y;
        g.y_stride[j] = p.act_row_bytes;
        g.nb[j] = p.K / 256;
        g.n_mat[j] = p.n_mat;
        g.w0[j] = waves;
        waves += p.M * (p.K / 256);
    }
    g.n = (int)segs.size();
    for (int j = g.n; j <= 8; j++) g.w0[j] = waves;
    st = ctx->launch("ghip_quantize_q8_K_segs", dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, g);
    if (st != GHIP_STATUS_SUCCESS) return st;
    ctx->hold = (total + 255) & ~(size_t)255;
    for (size_t gi = 0; gi < groups.size(); gi++) {
        if (seg_of[gi] < 0) continue;
        const Seg &sg = segs[seg_of[gi]];
        pre[gi] = (const uint8_t *)ws + sg.off;
        ghip_tensor &v = pre_view[gi];
        v = *sg.x;
        v.type = GHIP_TYPE_Q8_K;
        v.data = (void *)pre[gi];
        v.nb[0] = 292;
        v.nb[1] = (size_t)sg.p.act_row_bytes;
        v.nb[2] = v.nb[1] * (size_t)v.ne[1];
        v.nb[3] = v.nb[2];
    }
    return GHIP_STATUS_SUCCESS;
}

ghip_status ghip_graph_compute(ghip_context *ctx, const ghip_node *nodes, int32_t n_nodes, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    if (n_nodes < 0 || (n_nodes > 0 && !nodes))
        return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "graph_compute: bad node list");
    const bool fuse = env_int("GHIP_GRAPH_FUSE", 1) != 0;
    // the node groups: siblings run as one multi-matrix launch
    std::vector<std::pair<int, int>> groups;
    for (int i = 0; i < n_nodes;) {
        int next = i + 1;
        if (nodes[i].op == GHIP_OP_MUL_MAT && fuse && multi_candidate(nodes[i]))
            while (next < n_nodes && next - i < 4 && joins_group(nodes, i, next)) next++;
        groups.push_back({i, next});
        i = next;
    }
    std::vector<const uint8_t *> pre(groups.size(), nullptr);
    std::vector<ghip_tensor> pre_view(groups.size());
    ghip_status st = prequantize(ctx, nodes, groups, pre, pre_view, (hipStream_t)stream);
    if (st != GHIP_STATUS_SUCCESS) return st;
    struct Unhold {
        ghip_context *c;
        ~Unhold() { c->hold = 0; }
    } unhold{ctx};
    for (size_t gi = 0; gi < groups.size(); gi++) {
        const int i = groups[gi].first, next = groups[gi].second;
        const ghip_node &nd = nodes[i];
        switch (nd.op) {
        case GHIP_OP_MUL_MAT:
            if (next - i >= 2)
                st = nd.src[1]->ne[1] >= env_int("GHIP_GEMM_MIN_ROWS", 16)
                         ? mul_mat_multi_gemm(ctx, nodes + i, next - i, (hipStream_t)stream)
                         : mul_mat_multi(ctx, nodes + i, next - i, (hipStream_t)stream, pre[gi]);
            else
                st = ghip_mul_mat(ctx, nd.src[0], pre[gi] ? &pre_view[gi] : nd.src[1], nd.dst, stream);
            break;
        case GHIP_OP_MUL_MAT_ID:
            st = ghip_mul_mat_id(ctx, nd.src[0], nd.src[1], nd.src[2], nd.dst, stream);
            break;
        case GHIP_OP_FLASH_ATTN_EXT:
            st = ghip_flash_attn_ext(ctx, nd.src[0], nd.src[1], nd.src[2], nd.src[3], nd.src[4], nd.dst, stream);
            break;
        default:
            return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "graph_compute: node %d: op %d not supported", i, nd.op);
        }
        if (st != GHIP_STATUS_SUCCESS) return st;
    }
    return GHIP_STATUS_SUCCESS;
}

ghip_status ghip_set_workspace(ghip_context *ctx, void *ptr, size_t bytes) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (!ptr && bytes) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "set_workspace: null pointer with a size");
    ctx->user_ws = bytes ? ptr : nullptr;
    ctx->user_ws_size = bytes;
    return GHIP_STATUS_SUCCESS;
}

ghip_status ghip_workspace_size(int op, const ghip_tensor *dst, const ghip_tensor *const *srcs, int n_srcs,
                                size_t *bytes) {
    if (!bytes) return GHIP_STATUS_BACKEND_ERROR;
    *bytes = 0;
    ghip_context tmp;
    ghip_status st = GHIP_STATUS_BACKEND_ERROR;
    if (op == GHIP_OP_MUL_MAT) {
        if (n_srcs < 2 || !srcs || !dst) return st;
        MulMatPlan p;
        if (!plan_mul_mat(&tmp, srcs[0], srcs[1], dst, p, st)) return st;
        if (p.M == 0 || p.N == 0) return GHIP_STATUS_SUCCESS;
        *bytes = mul_mat_ws_bytes(p, true, false, nullptr, nullptr);
        return GHIP_STATUS_SUCCESS;
    }
    if (op == GHIP_OP_MUL_MAT_ID) {
        if (n_srcs < 3 || !srcs || !dst) return st;
        MoePlan p;
        if (!plan_moe(&tmp, srcs[0], srcs[1], srcs[2], dst, p, st)) return st;
        if (p.n_ids * p.n_tokens == 0 || p.rows == 0) return GHIP_STATUS_SUCCESS;
        *bytes = moe_ws(p, true, false).total;
        return GHIP_STATUS_SUCCESS;
    }
    if (op == GHIP_OP_FLASH_ATTN_EXT) {
        if (n_srcs < 3 || !srcs || !dst) return st;
        const ghip_tensor *q = srcs[0], *k = srcs[1], *v = srcs[2];
        if (!plan_fa(&tmp, q, k, v, n_srcs > 3 ? srcs[3] : nullptr, n_srcs > 4 ? srcs[4] : nullptr, dst, st)) return st;
        if (q->ne[1] == 0 || q->ne[2] == 0) return GHIP_STATUS_SUCCESS;
        const ghip_tensor *m = n_srcs > 3 ? srcs[3] : nullptr;
        *bytes = fa_layout((int)k->ne[0], (int)q->ne[1], (int)q->ne[2], (int)k->ne[1], (int)k->ne[2],
                           m ? (int)m->ne[2] : 0).ws_bytes;
        return GHIP_STATUS_SUCCESS;
    }
    return st;
}

ghip_status ghip_quantize_chunk(ghip_context *ctx, int type, const float *src, void *dst, int64_t nrows,
                                int64_t n_per_row, void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    std::lock_guard<std::mutex> lock(ctx->mu);
    const TypeInfo ti = type_info(type);
    const char *name = type == GHIP_TYPE_Q4_0   ? "ghip_wquant_q4_0"
                       : type == GHIP_TYPE_Q4_K ? "ghip_wquant_q4_K"
                       : type == GHIP_TYPE_Q6_K ? "ghip_wquant_q6_K"
                       : type == GHIP_TYPE_MXFP4 ? "ghip_wquant_mxfp4"
                                                 : nullptr;
    if (!name) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "quantize_chunk: type %d not supported", type);
    if (nrows < 0 || n_per_row <= 0 || n_per_row % ti.blck)
        return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "quantize_chunk: n_per_row %% block size != 0");
    if (!src || !dst) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "quantize_chunk: null pointer");
    const int64_t nblocks = nrows * (n_per_row / ti.blck);
    if (nblocks == 0) return GHIP_STATUS_SUCCESS;
    if (!ctx->set_device()) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    const unsigned tpb = ti.blck == 256 ? 64 : 256;
    const unsigned grid = (unsigned)((nblocks + tpb - 1) / tpb);
    return ctx->launch(name, dim3(grid), dim3(tpb), 0, (hipStream_t)stream, src, nblocks, (uint8_t *)dst);
}

}  // extern "C"
