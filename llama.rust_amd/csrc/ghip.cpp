// ghip.cpp -- host side of the gfx950 backend: code-object loading, operand
// validation, workspace management and kernel dispatch behind include/ghip.h.
#include "../../include/ghip.h"

#include <hip/hip_runtime.h>

#include <dlfcn.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

const char *const kModules[] = {"ghip_quant.hsaco", "ghip_gemv.hsaco", "ghip_wquant.hsaco", "ghip_gemm.hsaco"};

struct TypeInfo {
    int blck;
    int bytes;
};

TypeInfo type_info(int t) {
    switch (t) {
    case GHIP_TYPE_F32: return {1, 4};
    case GHIP_TYPE_F16: return {1, 2};
    case GHIP_TYPE_Q4_0: return {32, 18};
    case GHIP_TYPE_Q8_0: return {32, 34};
    case GHIP_TYPE_Q4_K: return {256, 144};
    case GHIP_TYPE_Q6_K: return {256, 210};
    case GHIP_TYPE_Q8_K: return {256, 292};
    case GHIP_TYPE_I32: return {1, 4};
    case GHIP_TYPE_MXFP4: return {32, 17};
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
    void *ws = nullptr;  // device workspace (quantized activations)
    size_t ws_size = 0;
    std::mutex mu;

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

    // grow-only workspace; waits for in-flight work before releasing the old one
    ghip_status workspace(size_t bytes, hipStream_t s, void **out) {
        if (bytes > ws_size) {
            if (ws) {
                hipStreamSynchronize(s);
                hipDeviceSynchronize();
                hipFree(ws);
                ws = nullptr;
                ws_size = 0;
            }
            const size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
            if (hipMalloc(&ws, want) != hipSuccess) {
                (void)hipGetLastError();
                return fail(GHIP_STATUS_OUT_OF_MEMORY, "workspace hipMalloc(%zu) failed", want);
            }
            ws_size = want;
        }
        *out = ws;
        return GHIP_STATUS_SUCCESS;
    }

    template <typename... Args>
    ghip_status launch(const std::string &name, dim3 grid, dim3 block, size_t shmem, hipStream_t s,
                       Args... args) {
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

bool plan_mul_mat(ghip_context *ctx, const ghip_tensor *a, const ghip_tensor *b, const ghip_tensor *d,
                  MulMatPlan &p, ghip_status &st) {
    st = GHIP_STATUS_BACKEND_ERROR;
    if (!a || !b) { st = ctx->fail(st, "mul_mat: null operand"); return false; }
    if (a->type != GHIP_TYPE_Q4_0 && a->type != GHIP_TYPE_Q4_K && a->type != GHIP_TYPE_Q6_K) {
        st = ctx->fail(st, "mul_mat: src0 type %d not supported (Q4_0, Q4_K, Q6_K)", a->type);
        return false;
    }
    const TypeInfo ti = type_info(a->type);
    const int vdt = a->type == GHIP_TYPE_Q4_0 ? GHIP_TYPE_Q8_0 : GHIP_TYPE_Q8_K;  // vec_dot_type
    if (b->type != GHIP_TYPE_F32 && b->type != vdt) {
        st = ctx->fail(st, "mul_mat: src1 must be F32 or the vec_dot type of src0 (backend.rs:2057-2066)");
        return false;
    }
    if (a->ne[0] != b->ne[0]) { st = ctx->fail(st, "mul_mat: ne00 != ne10"); return false; }
    if (a->ne[0] % ti.blck) { st = ctx->fail(st, "mul_mat: ne00 %% block size != 0"); return false; }
    if ((int64_t)a->nb[0] != ti.bytes) { st = ctx->fail(st, "mul_mat: permuted src0 (nb0 != type size)"); return false; }
    if ((int64_t)b->nb[0] != type_info(b->type).bytes) { st = ctx->fail(st, "mul_mat: permuted src1"); return false; }
    if (a->ne[2] != 1 || a->ne[3] != 1 || b->ne[2] != 1 || b->ne[3] != 1) {
        st = ctx->fail(st, "mul_mat: only 2-D operands are supported");
        return false;
    }
    if (b->type == GHIP_TYPE_F32 && b->nb[1] % 4) { st = ctx->fail(st, "mul_mat: src1 row stride not a multiple of 4"); return false; }
    if (d) {
        if (d->type != GHIP_TYPE_F32 || d->nb[0] != 4 || d->ne[0] != a->ne[1] || d->ne[1] != b->ne[1] ||
            d->nb[1] % 4) {
            st = ctx->fail(st, "mul_mat: dst must be F32 [ne01, ne11] with nb0 == 4");
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
    if (a->type == GHIP_TYPE_Q4_0) {
        p.act_type = GHIP_TYPE_Q8_0;
        p.act_row_bytes = p.K / 32 * 34;
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
    if (p.act_type == GHIP_TYPE_Q8_K) {
        const int64_t waves = p.M * (p.K / 256);
        const unsigned grid = (unsigned)((waves + 3) / 4);
        return ctx->launch("ghip_quantize_q8_K", dim3(grid), dim3(256), 0, s, (const float *)b->data, x_stride,
                           (int64_t)p.K, (int64_t)p.M, (uint8_t *)out, (int64_t)p.act_row_bytes, (int64_t)p.n_mat);
    }
    const int64_t blocks = p.M * (p.K / 32);
    const unsigned grid = (unsigned)((blocks * 8 + 255) / 256);
    return ctx->launch("ghip_quantize_q8_0", dim3(grid), dim3(256), 0, s, (const float *)b->data, x_stride,
                       (int64_t)p.K, (int64_t)p.M, (uint8_t *)out, (int64_t)p.act_row_bytes);
}

const char *gemv_base(int wtype) {
    switch (wtype) {
    case GHIP_TYPE_Q4_K: return "ghip_gemv_q4_K";
    case GHIP_TYPE_Q6_K: return "ghip_gemv_q6_K";
    default: return "ghip_gemv_q4_0";
    }
}

// Decode path: activation columns in groups of at most 8.
ghip_status run_gemv(ghip_context *ctx, const MulMatPlan &p, const void *w, const uint8_t *act, float *dst,
                     int64_t ldd, int32_t *sub, hipStream_t s) {
    int waves_k;
    if (p.wtype == GHIP_TYPE_Q4_0)
        waves_k = (int)(((p.nb + 1) / 2 + 63) / 64);
    else
        waves_k = (int)((p.nb + 7) / 8);
    if (waves_k > 8) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: ne00 = %lld too large for the decode kernel", (long long)p.K);
    const int rows_per_wg = 8;  // RB in ghip_gemv.hip
    const unsigned grid = (unsigned)((p.N + rows_per_wg - 1) / rows_per_wg);
    for (int64_t c0 = 0; c0 < p.M; c0 += 8) {
        const int nc = (int)std::min<int64_t>(8, p.M - c0);
        const int NC = nc == 1 ? 1 : nc == 2 ? 2 : nc <= 4 ? 4 : 8;
        std::string name = std::string(gemv_base(p.wtype)) + (sub ? "_sub" : "") + "_c" + std::to_string(NC);
        int32_t *sub_c = sub;
        if (sub) {
            const int64_t per = p.wtype == GHIP_TYPE_Q4_K ? 2 * p.nb : p.nb;
            sub_c = sub + c0 * p.N * per;
        }
        ghip_status st = ctx->launch(name, dim3(grid), dim3(64 * waves_k), 0, s, (const uint8_t *)w,
                                     (int64_t)p.w_row_bytes, (int)p.N, (int)p.nb, act + c0 * p.act_row_bytes,
                                     (int64_t)p.act_row_bytes, nc, dst + c0 * ldd, (int64_t)ldd, sub_c);
        if (st != GHIP_STATUS_SUCCESS) return st;
    }
    return GHIP_STATUS_SUCCESS;
}

// Prefill path (Q4_K, many activation rows): int8 MFMA GEMM, 128 x 128 tiles.
constexpr size_t kGemmSmem = 114176;  // sizeof(GemmSmem) in ghip_gemm.hip
ghip_status run_gemm(ghip_context *ctx, const MulMatPlan &p, const void *w, const uint8_t *act, float *dst,
                     int64_t ldd, int32_t *sub, hipStream_t s) {
    const unsigned grid = (unsigned)(((p.M + 127) / 128) * ((p.N + 127) / 128));
    return ctx->launch("ghip_gemm_q4_K", dim3(grid), dim3(256), kGemmSmem, s, (const uint8_t *)w,
                       (int64_t)p.w_row_bytes, (int)p.N, (int)p.nb, act, (int64_t)p.act_row_bytes, (int)p.M, dst,
                       (int64_t)ldd, sub);
}

bool use_gemm(const MulMatPlan &p) {
    const int min_m = env_int("GHIP_GEMM_MIN_ROWS", 16);
    return p.wtype == GHIP_TYPE_Q4_K && p.M >= min_m && p.M <= INT32_MAX;
}

ghip_status mul_mat_impl(ghip_context *ctx, const ghip_tensor *a, const ghip_tensor *b, const ghip_tensor *d,
                         int32_t *sub, void *act_out, void *stream) {
    std::lock_guard<std::mutex> lock(ctx->mu);
    MulMatPlan p;
    ghip_status st;
    if (!plan_mul_mat(ctx, a, b, d, p, st)) return st;
    hipStream_t s = (hipStream_t)stream;
    if (p.M == 0 || p.N == 0) return GHIP_STATUS_SUCCESS;  // empty operands: nothing to compute
    if (hipSetDevice(ctx->device) != hipSuccess) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    if (!d && !sub && !act_out) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: no output");
    // workspace: [quantized activations | f32 scratch output when only sub-sums are wanted]
    const size_t act_bytes = p.act_pre ? 0 : ((size_t)(p.M * p.act_row_bytes) + 255) & ~(size_t)255;
    const size_t need = (act_out ? 0 : act_bytes) + (d || act_out ? 0 : (size_t)(p.M * p.N * 4));
    void *ws = nullptr;
    if (need) {
        st = ctx->workspace(need, s, &ws);
        if (st != GHIP_STATUS_SUCCESS) return st;
    }
    void *act = act_out ? act_out : ws;
    if (p.act_pre) {
        if (act_out) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat_act: src1 is already quantized");
        act = b->data;
    } else {
        st = quantize_act(ctx, p, b, act, s);
        if (st != GHIP_STATUS_SUCCESS || act_out) return st;
    }
    float *dst = d ? (float *)d->data : (float *)((uint8_t *)ws + act_bytes);
    const int64_t ldd = d ? (int64_t)d->nb[1] / 4 : p.N;
    if (use_gemm(p)) return run_gemm(ctx, p, a->data, (const uint8_t *)act, dst, ldd, sub, s);
    return run_gemv(ctx, p, a->data, (const uint8_t *)act, dst, ldd, sub, s);
}

}  // namespace

extern "C" {

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

void ghip_free(ghip_context *ctx) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    hipDeviceSynchronize();
    if (ctx->ws) hipFree(ctx->ws);
    for (hipModule_t m : ctx->modules) hipModuleUnload(m);
    delete ctx;
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
    return 0;
}

ghip_status ghip_mul_mat(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1, const ghip_tensor *dst,
                         void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    if (!dst) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "mul_mat: null dst");
    return mul_mat_impl(ctx, src0, src1, dst, nullptr, nullptr, stream);
}

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
    if (hipSetDevice(ctx->device) != hipSuccess) return ctx->fail(GHIP_STATUS_BACKEND_ERROR, "hipSetDevice failed");
    const unsigned tpb = ti.blck == 256 ? 64 : 256;
    const unsigned grid = (unsigned)((nblocks + tpb - 1) / tpb);
    return ctx->launch(name, dim3(grid), dim3(tpb), 0, (hipStream_t)stream, src, nblocks, (uint8_t *)dst);
}

}  // extern "C"
