/*
 * ghip.h -- C ABI of the MI355X (gfx950) backend for llama.rust's quantized
 * ggml hot path: GGML_OP_MUL_MAT (Q4_0 / Q4_K / Q6_K weights),
 * GGML_OP_MUL_MAT_ID and GGML_OP_FLASH_ATTN_EXT (f16 / f32 K/V).
 *
 * The entry points are what a Rust `ggml-hip` FFI crate binds (one extern "C"
 * fn per declaration, no other glue); each comment names the reference
 * interface it replaces (paths relative to fly88oj/llama.rust).
 *
 * Conventions
 *  - Tensors are described with ggml's own geometry: ne[] in elements,
 *    innermost first; nb[] in bytes; data is a DEVICE pointer.  Block layouts
 *    are the GGUF ones, untouched (crates/ggml/src/blocks.rs:33-168).
 *  - stream is a hipStream_t (NULL = the legacy default stream).  Every
 *    compute call is asynchronous on that stream.
 *  - Errors are returned as ghip_status (the values of enum ggml_status,
 *    crates/ggml/src/backend.rs:54-62); ghip_last_error() explains the last
 *    failure of a context.  Nothing falls back to the CPU: an unsupported
 *    shape or type returns GHIP_STATUS_BACKEND_ERROR.
 *  - A context may be used from any host thread; calls are serialised.
 *  - Scratch memory (quantized activations, GEMM layouts, split partials,
 *    routing tables) comes from one workspace per context.  By default the
 *    library owns it and grows it on demand with hipMalloc; a call that would
 *    grow it while its stream is being captured fails with
 *    GHIP_STATUS_ALLOC_FAILED instead (run the call once before capturing, or
 *    give a workspace with ghip_set_workspace).  Outgrown buffers are kept
 *    until ghip_free, so graphs captured earlier stay valid.  A call on a
 *    different stream than the previous call first waits for the previous
 *    stream (an event), so two streams never use the workspace at once; when
 *    either stream is being captured that wait cannot be recorded and the
 *    caller orders the streams.
 */
#ifndef GHIP_H
#define GHIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* enum ggml_status (crates/ggml/src/backend.rs:54-62) */
typedef enum ghip_status {
    GHIP_STATUS_SUCCESS = 0,
    GHIP_STATUS_ALLOC_FAILED = 1,
    GHIP_STATUS_OUT_OF_MEMORY = 2,
    GHIP_STATUS_BACKEND_ERROR = 3,
    GHIP_STATUS_ABORTED = 4,
} ghip_status;

/* enum ggml_type ids (crates/ggml/src/types.rs:15) for the types this
 * backend reads or writes */
enum {
    GHIP_TYPE_F32 = 0,
    GHIP_TYPE_F16 = 1,
    GHIP_TYPE_Q4_0 = 2,
    GHIP_TYPE_Q4_1 = 3,
    GHIP_TYPE_Q5_0 = 6,
    GHIP_TYPE_Q5_1 = 7,
    GHIP_TYPE_Q8_0 = 8,
    GHIP_TYPE_Q8_1 = 9,
    GHIP_TYPE_Q2_K = 10,
    GHIP_TYPE_Q3_K = 11,
    GHIP_TYPE_Q4_K = 12,
    GHIP_TYPE_Q5_K = 13,
    GHIP_TYPE_Q6_K = 14,
    GHIP_TYPE_Q8_K = 15,
    GHIP_TYPE_IQ4_NL = 20,
    GHIP_TYPE_IQ4_XS = 23,
    GHIP_TYPE_I32 = 26,
    GHIP_TYPE_IQ2_XXS = 16,
    GHIP_TYPE_IQ2_XS = 17,
    GHIP_TYPE_IQ3_XXS = 18,
    GHIP_TYPE_IQ1_S = 19,
    GHIP_TYPE_IQ3_S = 21,
    GHIP_TYPE_IQ2_S = 22,
    GHIP_TYPE_IQ1_M = 29,
    GHIP_TYPE_BF16 = 30,
    GHIP_TYPE_MXFP4 = 39,
    GHIP_TYPE_NVFP4 = 40,
    GHIP_TYPE_Q1_0 = 41,
    GHIP_TYPE_Q2_0 = 42,
};

/* The ops of the hot path (GgmlOp::MulMat / MulMatId / FlashAttnExt,
 * crates/ggml/src/ops.rs:1329, :1421, :2430). */
enum {
    GHIP_OP_MUL_MAT = 1,
    GHIP_OP_MUL_MAT_ID = 2,
    GHIP_OP_FLASH_ATTN_EXT = 3,
};

/* The subset of struct ggml_tensor the kernels read
 * (GgmlCTensor, crates/ggml/src/sysffi.rs:212-228; TensorMeta tensor.rs:295-309). */
typedef struct ghip_tensor {
    int32_t type;
    int64_t ne[4];
    uint64_t nb[4];
    void *data;            /* device pointer */
    int32_t op_params[16]; /* FLASH_ATTN_EXT: [0] scale, [1] max_bias, [2] softcap as f32 bits */
} ghip_tensor;

typedef struct ghip_context ghip_context;

/* Open the backend on HIP device `device`: loads the gfx950 code objects
 * (hipModuleLoad) that sit next to this library.
 * Replaces BackendDeviceI.init_backend (crates/ggml/src/backend.rs:966) /
 * the dlopen entry ggml_backend_init (backend.rs:1354-1420). */
ghip_status ghip_init(int device, ghip_context **out);

/* A context without a device, for checking launch plans on a host with no
 * GPU.  No counterpart in the reference (its CPU backend has no launches).
 * Ops on it plan their launches, take a workspace address range nothing
 * allocates and, instead of launching, check that every kernel's store
 * window (worked out from that launch's own arguments) lies inside the
 * buffers the op writes: its dst, sub-sum and activation outputs and the
 * workspace.  A window outside them fails the op with a "store check"
 * message.  Device pointers in the tensors are only compared, never read.
 * (GHIP_CHECK_STORES=1 in the environment makes ghip_init contexts run the
 * same check before their real launches.)  Free with ghip_free. */
ghip_status ghip_init_dry_run(ghip_context **out);

/* Release the context (BackendI.free, backend.rs:666). */
void ghip_free(ghip_context *ctx);

/* Human-readable reason of the last non-success status on ctx ("" if none). */
const char *ghip_last_error(const ghip_context *ctx);

/* Wait for all work queued through ctx on `stream` (BackendI.synchronize,
 * backend.rs:662). */
ghip_status ghip_synchronize(ghip_context *ctx, void *stream);

/* Capability check: 1 when the op with these operands runs on this backend,
 * else 0.  srcs are the op's sources in ggml order (MUL_MAT: src0, src1;
 * MUL_MAT_ID: as, b, ids; FLASH_ATTN_EXT: q, k, v, mask|NULL, sinks|NULL).
 * Replaces BackendDeviceI.supports_op (backend.rs:980, CPU semantics
 * backend.rs:2037-2071). */
int ghip_supports_op(int op, const ghip_tensor *dst, const ghip_tensor *const *srcs, int n_srcs);

/* dst = src0 x src1 (GGML_OP_MUL_MAT, forward_mul_mat compute.rs:1420-1839).
 * src0: Q4_0 | Q4_1 | Q5_0 | Q5_1 | Q8_0 | Q2_K | Q3_K | Q4_K | Q5_K | Q6_K |
 *       IQ4_NL | IQ4_XS | NVFP4 | Q1_0 | Q2_0 | IQ1_S | IQ1_M | IQ2_XXS | IQ2_XS | IQ2_S |
 *       IQ3_XXS | IQ3_S weight [ne00=K, ne01=N, ne02, ne03], rows contiguous;
 *       or F32 | F16 | BF16 weight [ne00=K, ne01=N, ne02, ne03] (src1 must then be F32:
 *       the activations are rounded to the weight type, compute.rs:1680-1745; no sub-sums)
 * src1: F32 [K, ne11, ne12, ne13] (any strides nb11..nb13, nb10 == 4), or
 *       already the vec_dot type of src0 (Q8_0 for Q4_0/Q5_0/Q8_0/IQ4_NL/NVFP4/Q1_0/Q2_0,
 *       Q8_1 for Q4_1/Q5_1, Q8_K for the K-quants and IQ4_XS; rows of blocks),
 *       which skips the quantization (backend.rs:2057-2066 semantics);
 * dst:  F32 [N, ne11, ne12, ne13] (nb0 == 4).
 * Planes: ne12 % ne02 == 0 and ne13 % ne03 == 0; dst plane (i12, i13) is
 * src0 plane (i12 / r2, i13 / r3) times src1 plane (i12, i13), r2 = ne12 /
 * ne02, r3 = ne13 / ne03 (compute.rs:1440-1450), each plane a 2-D MUL_MAT
 * (sub-sums and quantized activations of the hooks below follow one another
 * plane by plane, i13 outermost).
 * Activations are quantized on the device exactly as the reference's route for
 * this (type, N, ne11) does (Q8_0 for Q4_0/Q5_0/Q8_0; Q8_1 for Q4_1/Q5_1,
 * quantize_row_q8_1 quants.rs:375; Q8_K for the K-quants, with the
 * quantize_mat_q8_K_4x8 values for the leading ne11 - ne11 % 4 rows of a
 * repacked Q4_K, compute.rs:5350-5398). */
ghip_status ghip_mul_mat(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1,
                         const ghip_tensor *dst, void *stream);

/* ghip_mul_mat without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * operands, kernels and results as ghip_mul_mat; the scratch is a fixed
 * 32 MiB array in this library's code object, one per GPU, held until the
 * process ends.  A call needing more scratch (e.g. the Q6_K prefill GEMM's
 * per-call weight repack of a large matrix) fails with
 * GHIP_STATUS_ALLOC_FAILED.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other contexts) race. */
ghip_status ghip_mul_mat_noalloc(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1,
                                 const ghip_tensor *dst, void *stream);

/* Parity hook with no reference counterpart (the reference exposes these
 * integers only inside its kernels, e.g. repack.rs:1664-1680): writes the exact
 * int32 partials ghip_mul_mat forms, per (activation row c, weight row r,
 * block b), at subsums[(c*N + r)*P + ...]:
 *   Q4_K, Q5_K: P = 2*nb, {iacc, imin} of super-block b
 *   Q6_K: P = nb,   sum_s scale_s * sum (q6-32)*q8 of super-block b
 *   Q4_0: P = nb,   sum (nib-8)*q8 of 32-block b
 *   Q5_0: P = nb,   sum ((nib | hbit << 4) - 16)*q8 of 32-block b
 *   Q8_0: P = nb,   sum q8w*q8 of 32-block b
 *   IQ4_NL: P = nb, sum kvalue*q8 of 32-block b
 *   NVFP4: P = 4*nb, sum kvalue*q8 of each 16-element sub-block of 64-block b
 *   IQ4_XS: P = nb, sum_g (ls_g - 32) * sum kvalue*q8 of super-block b
 *   Q1_0: P = 4*nb, Q2_0: P = 2*nb, sum value*q8 of each 32-element group
 *   IQ1 / IQ2 / IQ3: P = nb, per super-block sum over its 32-element blocks of
 *     scale * sum value*q8 (IQ1: value = 8 * grid + delta), the integer
 *     the reference's tiled kernel scales
 * subsums is a device pointer of ne11*N*P int32. */
ghip_status ghip_mul_mat_subsums(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1,
                                 int32_t *subsums, void *stream);

/* Parity hook with no reference counterpart: the activation blocks
 * ghip_mul_mat feeds its kernels for (src0, src1) -- ne11 plain rows of
 * block_q8_0 (Q4_0, Q5_0, Q8_0), block_q8_1 (Q4_1, Q5_1) or block_q8_K (the K-quants) -- written to the device
 * pointer out.  Same quantizers as compute.rs:1504-1549 / :5350-5398. */
ghip_status ghip_mul_mat_act(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1,
                             void *out, void *stream);

/* dst = MUL_MAT_ID(as, b, ids) with MXFP4, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0,
 * Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS, NVFP4, Q1_0 or Q2_0 experts
 * (forward_mul_mat_id, compute.rs:1917-2202; the MXFP4 rows % 8 == 0 repack
 * kernel repack.rs:1048-1100):
 *   as:  [K, rows, n_as], expert rows contiguous blocks
 *   b:   F32 [K, ne11, n_tokens] (nb0 == 4, nb2 == ne11 * nb1), 1 <= ne11 <= n_ids
 *   ids: I32 [n_ids, n_tokens], expert index per (slot, token)
 *   dst: F32 [rows, n_ids, n_tokens] (nb0 == 4)
 * MXFP4: dst[t][s] = as[ids[t][s]] x quantize_q8_0(b[t][s % ne11]).  Each
 * 32-block dot is exact and folded in block order with the reference's own
 * operations (fma(dot, e * d, acc) for rows % 8 == 0, acc += (d * e) * dot
 * otherwise), so outputs are bit-identical.
 * Q4_K / Q5_K / Q6_K (K % 256 == 0): the same with quantize_row_q8_K
 * activations (compute.rs:1950-1980); each super-block's integer sums are
 * exact and scaled once by d8 * d (vec_dot.rs:881-909, :998-1028), so outputs
 * match the reference's routes to fp32 rounding of those per-block terms.
 * The other types: every b row quantized to the type's vec_dot type
 * (Q8_0, Q8_1 or Q8_K, compute.rs:1950-1976), then per pair the expert's
 * decode kernel of ghip_mul_mat (the reference's row vec_dot, Q4_0's 8x8
 * repack gemv, or for Q2_K / Q3_K / IQ4_XS experts with >= 8 pairs its tiled
 * kernel: the same integer sums, fp32 within rounding of their order).
 * A pair whose id is outside [0, n_as) -- where the reference asserts -- gets
 * a row of NaN. */
ghip_status ghip_mul_mat_id(ghip_context *ctx, const ghip_tensor *as, const ghip_tensor *b, const ghip_tensor *ids,
                            const ghip_tensor *dst, void *stream);

/* Parity hook with no reference counterpart: the int32 partials that
 * ghip_mul_mat_id folds (device pointer), per (pair p = t * n_ids + s, row r):
 *   MXFP4: the block dots sum kvalue * q8 at subsums[(p * rows + r) * (K / 32) + block];
 *   Q4_K / Q5_K: (sum sc * dot, sum m * bsum) per super-block at
 *     subsums[((p * rows + r) * (K / 256) + sb) * 2 + {0, 1}];
 *   Q6_K: sum sc * (dot - 32 * bsum) per super-block at
 *     subsums[(p * rows + r) * (K / 256) + sb]
 *   other types: the ghip_mul_mat_subsums row of the type, P ints per row at
 *     subsums[(p * rows + r) * P + j]
 * (the layouts of ghip_mul_mat_subsums).  Pairs with an invalid id are left
 * unwritten. */
ghip_status ghip_mul_mat_id_subsums(ghip_context *ctx, const ghip_tensor *as, const ghip_tensor *b,
                                    const ghip_tensor *ids, int32_t *subsums, void *stream);

/* dst = FLASH_ATTN_EXT(q, k, v, mask, sinks) (forward_flash_attn_ext
 * compute.rs:4563-4625; FlashAttn flash_attn.rs:273-386):
 *   q:     F32 [DK, T, H, n_seq]      (nb0 == 4, any nb1..nb3)
 *   k:     F16 or F32 [DK, S, H_kv, n_seq], v: F16 or F32 [DV, S, H_kv, n_seq]
 *          (rows contiguous), DK and DV in 1..256, H % H_kv == 0
 *          (flash_attn.rs:298-313)
 *   mask:  F16 [>= S, >= T, m2, m3] or NULL (rows contiguous); head h of
 *          sequence i3 reads plane (h % m2, i3 % m3), H % m2 == 0 and
 *          n_seq % m3 == 0 (ggml.c:5517-5518, flash_attn.rs:30-37)
 *   sinks: F32 [H] or NULL
 *   dst:   F32 [DV, H, T, n_seq], each sequence contiguous
 *   dst->op_params: [0] scale, [1] max_bias, [2] logit_softcap (f32 bits).
 * F16 K/V with DK == DV in {64, 128} and H / H_kv <= 8 run the matrix-core
 * kernels (the KV range split across workgroups and merged in slice order);
 * every other shape runs a row walk in key order (the reference's attn_row,
 * with its f16 accumulator for an F16 V on that route); so does a
 * single-query split-KV shape with per-head mask planes.  Sequences run one
 * after another.  The result matches the reference within 2e-3 max-abs. */
ghip_status ghip_flash_attn_ext(ghip_context *ctx, const ghip_tensor *q, const ghip_tensor *k, const ghip_tensor *v,
                                const ghip_tensor *mask, const ghip_tensor *sinks, const ghip_tensor *dst,
                                void *stream);

/* One node of a graph: the op, its sources in ggml order (MUL_MAT: src0,
 * src1; MUL_MAT_ID: as, b, ids; FLASH_ATTN_EXT: q, k, v, mask|NULL,
 * sinks|NULL; unused slots NULL) and its destination
 * (ggml_tensor.op / src[] / the node itself, GgmlCTensor sysffi.rs:212-228). */
typedef struct ghip_node {
    int32_t op; /* GHIP_OP_* */
    const ghip_tensor *src[5];
    const ghip_tensor *dst;
} ghip_node;

/* Compute the nodes in order on stream, each exactly as its single-op entry
 * point above does (BackendI.graph_compute, crates/ggml/src/backend.rs:652-668
 * -> cpu_backend_graph_compute backend.rs:2169 -> compute::graph_compute
 * compute.rs:307).  Consecutive MUL_MAT nodes with 1-8 F32 activation rows
 * (Q6_K: one) that read the same src1 (same data and geometry) with the same
 * weight type (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K) and the same K -- a
 * layer's q/k/v or gate/up at decode -- run as one launch of up to four
 * matrices (Q4_0 / Q5_0 / Q8_0 after one Q8_0 quantization), provided
 * no node of the group reads or overlaps another's dst (and, for Q4_K at 4+
 * rows, N % 8 == 0 holds for all or none: it selects the activation
 * quantizer); their results are bit-identical to the single-op calls.
 * Q4_K siblings with prefill batches (the GEMM's range, 16+ rows) likewise
 * run as one GEMM launch over all their tiles after one activation
 * quantization; results match the single-op calls within the MUL_MAT
 * tolerance (a small matrix alone sums split-K slices in order).  Returns the first failing node's status (the nodes before
 * it have been enqueued); ghip_last_error names the failure.
 * GHIP_GRAPH_FUSE=0 in the environment turns the grouping off. */
ghip_status ghip_graph_compute(ghip_context *ctx, const ghip_node *nodes, int32_t n_nodes, void *stream);

/* Give the context caller-owned device memory as its workspace (no reference
 * counterpart: the reference's CPU ops allocate their quantized-activation
 * buffer inside each op, e.g. the wdata of forward_mul_mat, compute.rs:1499-1530).  From then on the context never
 * allocates; a call that needs more than `bytes` fails with
 * GHIP_STATUS_ALLOC_FAILED.  ptr = NULL, bytes = 0 returns to the owned
 * workspace.  The memory must stay valid while queued work or captured graphs
 * use it. */
ghip_status ghip_set_workspace(ghip_context *ctx, void *ptr, size_t bytes);

/* Workspace bytes one op needs (same operands as ghip_supports_op; dst is
 * required), pure host arithmetic with no reference counterpart (there the
 * size is implicit in each op's wdata, compute.rs:1499-1530).  For a node list, the maximum over its nodes is
 * enough for ghip_graph_compute (grouped launches need no more than their
 * members alone). */
ghip_status ghip_workspace_size(int op, const ghip_tensor *dst, const ghip_tensor *const *srcs, int n_srcs,
                                size_t *bytes);

/* Declare `w` (a 2-D weight in device memory, GGUF block layout) immutable
 * and keep device-side copies of it in the layouts the kernels read, built
 * once on `stream` now instead of on every call -- the reference's repack
 * cache (repack_*_cached, crates/ggml/src/repack.rs:4250-4480, and the
 * CPU_REPACK buffer it stands for).  Today those are the Q6_K prefill
 * GEMM's aligned 336-byte records, the Q4_0 / Q5_0 / Q8_0 prefill GEMM's
 * int8 code plane with its f32 block scales, and (3-D MXFP4 expert weights)
 * the MUL_MAT_ID kernel's 80-byte windows; other types are read in their
 * GGUF layout and register as a no-op.  Later MUL_MAT calls whose src0 has the same data
 * pointer, type, ne[0], ne[1] and nb[1] use the copy.  The same switches as
 * the reference: LLAMA_RUST_REPACK=0 turns it off, LLAMA_RUST_REPACK_MAX_MB
 * caps the bytes kept (default 16384); a weight over the cap is not kept and
 * calls repack it per call as before (both return success).  Allocates
 * (hipMalloc): fails with GHIP_STATUS_ALLOC_FAILED while `stream` is being
 * captured.  The weight's bytes must not change until
 * ghip_weight_unregister. */
ghip_status ghip_weight_register(ghip_context *ctx, const ghip_tensor *w, void *stream);

/* Drop the copies kept for `w` (waits for the device first, so queued work
 * that reads them completes).  Unknown weights are a no-op. */
ghip_status ghip_weight_unregister(ghip_context *ctx, const ghip_tensor *w);

/* Copies kept, their bytes, and how many were built so far (hits do not
 * count) -- repack_stats (repack.rs:4329-4334).  Any pointer may be NULL. */
ghip_status ghip_weight_cache_stats(ghip_context *ctx, size_t *n_weights, size_t *bytes, size_t *built);

/* ---- GGUF files (crates/ggml/src/gguf.rs:388-655, a port of
 * gguf_init_from_file): the container is memory-mapped and parsed on the
 * host; tensors are uploaded to device memory in their GGUF block layout
 * and, if asked, registered (ghip_weight_register) so their repacked copies
 * are built on the device once. */
typedef struct ghip_gguf ghip_gguf;

/* enum gguf_type (gguf.rs:49-63) */
enum {
    GHIP_GGUF_UINT8 = 0, GHIP_GGUF_INT8 = 1, GHIP_GGUF_UINT16 = 2, GHIP_GGUF_INT16 = 3,
    GHIP_GGUF_UINT32 = 4, GHIP_GGUF_INT32 = 5, GHIP_GGUF_FLOAT32 = 6, GHIP_GGUF_BOOL = 7,
    GHIP_GGUF_STRING = 8, GHIP_GGUF_ARRAY = 9, GHIP_GGUF_UINT64 = 10, GHIP_GGUF_INT64 = 11,
    GHIP_GGUF_FLOAT64 = 12,
};

/* TensorInfo (gguf.rs:211-228): nb computed from the type as gguf.cpp does;
 * offset relative to its part's data section; part = the split file. */
typedef struct ghip_gguf_tensor_info {
    char name[64];
    int32_t type;
    int64_t ne[4];
    uint64_t nb[4];
    uint64_t offset;
    uint64_t size;
    int32_t part;
} ghip_gguf_tensor_info;

/* Gguf::open (follow_splits != 0: the split.* pass, gguf.rs:388-480) or
 * Gguf::open_single.  On failure returns GHIP_STATUS_BACKEND_ERROR and the
 * reference's GgufError text (gguf.rs:278-300) in err. */
ghip_status ghip_gguf_open(const char *path, int follow_splits, ghip_gguf **out, char *err, size_t err_len);
void ghip_gguf_close(ghip_gguf *g);
uint32_t ghip_gguf_version(const ghip_gguf *g);
uint64_t ghip_gguf_alignment(const ghip_gguf *g);
uint64_t ghip_gguf_data_offset(const ghip_gguf *g);   /* part 0's */
int64_t ghip_gguf_n_parts(const ghip_gguf *g);
int64_t ghip_gguf_n_kv(const ghip_gguf *g);
const char *ghip_gguf_key(const ghip_gguf *g, int64_t i);
int64_t ghip_gguf_find_key(const ghip_gguf *g, const char *key);  /* -1 if absent */
int32_t ghip_gguf_kv_type(const ghip_gguf *g, int64_t i);         /* GHIP_GGUF_* */
int32_t ghip_gguf_arr_type(const ghip_gguf *g, int64_t i);        /* element type, -1 if not an array */
int64_t ghip_gguf_arr_n(const ghip_gguf *g, int64_t i);           /* element count, -1 if not an array */
/* Value of kv i (j = -1) or of element j of array kv i; 1 on success, 0 if
 * absent or of another type.  u32 / f32 follow Value::as_u32 / as_f32
 * (gguf.rs:141-168), u16 the exact type (as_u16); i64 reads any integer. */
int ghip_gguf_get_u32(const ghip_gguf *g, int64_t i, int64_t j, uint32_t *out);
int ghip_gguf_get_u16(const ghip_gguf *g, int64_t i, int64_t j, uint16_t *out);
int ghip_gguf_get_f32(const ghip_gguf *g, int64_t i, int64_t j, float *out);
int ghip_gguf_get_i64(const ghip_gguf *g, int64_t i, int64_t j, int64_t *out);
int ghip_gguf_get_f64(const ghip_gguf *g, int64_t i, int64_t j, double *out);
int ghip_gguf_get_bool(const ghip_gguf *g, int64_t i, int64_t j, int *out);
int ghip_gguf_get_str(const ghip_gguf *g, int64_t i, int64_t j, const char **s, size_t *n);
int64_t ghip_gguf_n_tensors(const ghip_gguf *g);
int64_t ghip_gguf_find_tensor(const ghip_gguf *g, const char *name);
ghip_status ghip_gguf_tensor(const ghip_gguf *g, int64_t i, ghip_gguf_tensor_info *out);
/* host pointer to tensor i's bytes in its part's mapping (tensor_data,
 * gguf.rs:632-640); NULL when they lie outside the file */
const void *ghip_gguf_tensor_data(const ghip_gguf *g, int64_t i);
/* Copy tensor i's bytes to the device pointer dst (at least its size) on
 * `stream` through pinned staging; returns when the copy is complete.  With
 * register_weight != 0 the uploaded tensor is then registered
 * (ghip_weight_register) and that build completes too. */
ghip_status ghip_gguf_upload(ghip_context *ctx, const ghip_gguf *g, int64_t i, void *dst, int register_weight,
                             void *stream);

/* Quantize nrows rows of n_per_row f32 values (device pointer src) into
 * GGUF blocks of `type` (Q4_0, Q4_K, Q6_K, MXFP4) at the device pointer dst,
 * byte-identical to the reference's no-imatrix quantizers
 * (ggml_quantize_chunk, crates/tools/quantize/src/rows.rs:63 ->
 * quantize_row_q4_0_ref quants.rs:124, quantize_row_q4_K_ref
 * quants_k.rs:1861, quantize_row_q6_K_ref quants_k.rs:2058; MXFP4 follows
 * upstream ggml's quantize_row_mxfp4_ref, which the reference lacks). */
ghip_status ghip_quantize_chunk(ghip_context *ctx, int type, const float *src, void *dst, int64_t nrows,
                                int64_t n_per_row, void *stream);

#ifdef __cplusplus
}
#endif
#endif
