// ghip_fa.hip -- GGML_OP_FLASH_ATTN_EXT with f16 K/V on the f16 matrix cores
// (v_mfma_f32_32x32x16_f16), online softmax in fp32.
//
// Semantics (flash_attn.rs:273-386, compute.rs:4563-4625): for query row t of
// head h,  s_k = scale * q.k  (softcap: s = softcap * tanh(s), scale being
// pre-divided by softcap), s_k += slope_h * mask[t][k]; out = softmax(s) V,
// rows whose keys are all masked give 0; sinks enter the softmax denominator
// as one extra logit per head.
//
// Work layout.  A workgroup owns one KV head hk, 32 * QS query positions and
// one slice of the KV range; its G * QS wavefronts are the G = H / H_kv query
// heads that share hk (GQA) times QS = ceil(4 / G) tiles of 32 queries, so
// every K/V tile staged in LDS serves >= 4 wavefronts.
// The next tile's K, V and mask values are loaded into registers while the
// current one is computed, and staged into the second of two LDS buffers
// after it (one barrier per tile).  Per
// 64-key tile each wavefront computes S^T = K Q^T (keys x queries), which
// leaves all scores of one query in one lane pair (l, l^32): the row max and
// row sum need one cross-lane exchange.  O^T += V^T P^T accumulates in 4 x 16
// fp32 registers per lane (DV = 128).  The KV range is split over
// workgroups (grid.z) so decode (1 query) and prefill both fill the GPU; the
// per-slice (M, S, O) partials are merged in slice order by ghip_fa_merge,
// exactly the reference's reduce_partials arithmetic shape (flash_attn.rs:779).
#include "ghip_common.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef __fp16 v4fp16 __attribute__((__vector_size__(8)));  // the transposing LDS read's type
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int FA_BQ = 32;   // query positions per workgroup
constexpr int FA_BK = 64;   // keys per tile
constexpr int FA_KPAD = 8;  // K row padding (halfs): 272-byte rows, 8 lanes' 16-byte reads hit distinct banks
constexpr int FA_VPAD = 4;  // V^T row padding (halfs) of the row walk's tiles
// prefill V tiles stay in key-major order, rows padded by 32 halfs (a row
// stride of 64 mod 256 bytes), so the 32 lanes of a transposing read
// (4 key rows x 4 dim groups x 2 dim halves) hit distinct banks
constexpr int FA_VNPAD = 32;

DEV int crow32(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

struct FaParams {
    const float *q;
    int64_t q_nb1, q_nb2;  // floats
    const uint16_t *k, *v;
    int64_t k_nb1, k_nb2, v_nb1, v_nb2;  // halfs
    const uint16_t *mask;
    int64_t mask_nb1;  // halfs
    int64_t mask_nb2;  // halfs: head h reads mask plane h % mask_ne2 (flash_attn.rs:30-37)
    int mask_ne2;
    float *dst;        // [T][H][DV]
    float *part;       // [(t*H + h)*nsplit + z][2 + DV]
    const float *sinks;  // [H] or null
    int T, S, H, H_kv, nsplit, chunk;
    float scale, softcap, m0, m1;
    int n_head_log2;
    int DK, DV;          // head sizes (the general kernel; the others are compiled per D)
    int k_f32, v_f32;    // K / V element type: 1 = F32 (strides still counted in halfs)
    // per (mask plane, 32-query block, 64-key tile): 0 every value +-0, 2 every
    // value -inf, 1 otherwise (ghip_fa_mask_scan); null: no flags
    const uint8_t *mflags;
    int nqb, ntile;
    // prefill over one KV slice (nsplit == 1): write the normalized output
    // instead of a partial for ghip_fa_merge_rows
    int direct;
};

DEV float head_slope(const FaParams &p, int h) {
    if (p.m0 == 1.0f && p.m1 == 1.0f) return 1.0f;
    // max_bias > 0: m0^(h+1) for h < n_head_log2 else m1^(2(h-n)+1)
    const float base = h < p.n_head_log2 ? p.m0 : p.m1;
    int e = h < p.n_head_log2 ? h + 1 : 2 * (h - p.n_head_log2) + 1;
    float r = 1.0f, a = base;
    while (e) {
        if (e & 1) r *= a;
        e >>= 1;
        if (e) a *= a;
    }
    return r;
}

template <int D, bool SOFTCAP>
__device__ __forceinline__ void fa_fwd_body(const FaParams &p, _Float16 *Ks2, _Float16 *Vn2) {
    constexpr int KS = D + FA_KPAD, VSN = D + FA_VNPAD;
    // 16-byte LDS chunks per key row (data and padding): one buffer-to-LDS
    // load of a wavefront fills 64 consecutive chunks, so a tile takes NIK (K)
    // and NIV (V) of them, spread over the workgroup's wavefronts (>= 4)
    constexpr int NIK = KS / 8, NIV = VSN / 8;
    constexpr int MKI = (NIK + 3) / 4, MVI = (NIV + 3) / 4;
    constexpr float LOG2E = 1.4426950408889634f;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nthr = blockDim.x;
    const int G = p.H / p.H_kv, QS = (nthr >> 6) / G;  // QS query tiles of 32 per workgroup
    // 1-D grid over (qt, hk, z), qt fastest.  Workgroups go to the 8 XCDs
    // round-robin; remap so that each XCD takes a contiguous run of ids and
    // the query tiles reading one K/V slice share that XCD's L2.
    const int qtiles = (p.T + FA_BQ * QS - 1) / (FA_BQ * QS);
    const int nwg = gridDim.x;
    const int bid = (nwg & 7) ? (int)blockIdx.x : (int)(blockIdx.x & 7) * (nwg >> 3) + (int)(blockIdx.x >> 3);
    const int qt = bid % qtiles, hk = (bid / qtiles) % p.H_kv, z = bid / (qtiles * p.H_kv);
    const int h = hk * G + w % G;
    const int li = lane & 31, h2 = lane >> 5;
    const int t = (qt * QS + w / G) * FA_BQ + li;  // this lane's query position
    const bool tvalid = t < p.T;
    const float slope = head_slope(p, h);
    // scores are kept in log2 units: s2 = log2(e) * (scale q.k + slope mask)
    const float sl2 = p.scale * LOG2E, ml2 = slope * LOG2E;

    // Q fragment (B operand of S^T = K Q^T): d = 16*kk + 8*h2 + 0..7
    v8h qf[D / 16];
    {
        const float *qr = p.q + (int64_t)h * p.q_nb2 + (int64_t)(tvalid ? t : 0) * p.q_nb1;
#pragma unroll
        for (int kk = 0; kk < D / 16; kk++)
#pragma unroll
            for (int e = 0; e < 8; e++) qf[kk][e] = tvalid ? (_Float16)qr[16 * kk + 8 * h2 + e] : (_Float16)0.0f;
    }
    v16f o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[dt][v] = 0.0f;
    // m_ref: reference max (log2 units, -inf until the first unmasked key);
    // mneg = -m_ref, or 0 while unset
    float m_ref = -__builtin_inff(), mneg = 0.0f, l_run = 0.0f;

    const int kb = z * p.chunk;
    const int ke = min(p.S, kb + p.chunk);
    const uint16_t *kbase = p.k + (int64_t)hk * p.k_nb2;
    const uint16_t *vbase = p.v + (int64_t)hk * p.v_nb2;
    // this wavefront's head reads mask plane h % mask_ne2 (wave-uniform)
    const int mplane_i = __builtin_amdgcn_readfirstlane(h % p.mask_ne2);
    const uint16_t *mplane = p.mask ? p.mask + (int64_t)mplane_i * p.mask_nb2 : nullptr;
    const uint16_t *mrow = mplane ? mplane + (int64_t)(tvalid ? t : 0) * p.mask_nb1 : nullptr;
    // mask tile classes of this wavefront's query block, 64 tiles per window:
    // lane l holds tile (window base + l)
    const uint8_t *mfl = p.mflags && mrow ? p.mflags + ((int64_t)mplane_i * p.nqb + (qt * QS + w / G)) * p.ntile : nullptr;
    int fl_base = -64, fl_win = 1;
    auto tile_class = [&](int tile) {  // tile: key tile index k0 / 64 (uniform, increasing)
        if (tile >= fl_base + 64) {
            fl_base = tile;
            fl_win = fl_base + lane < p.ntile ? (int)mfl[fl_base + lane] : 1;
        }
        return __builtin_amdgcn_readlane(fl_win, tile - fl_base);
    };

    // Next tile in registers while this one is computed: K chunks, V blocks of
    // 4 keys x 8 dims (transposed on the way into LDS), and this lane's mask
    // values (keys 32*jt + 8*gq + 4*h2 + 0..3, the layout of the scores).
    uint2 mr[2][4], mrn[2][4];  // this tile's and the next tile's mask values
#pragma unroll
    for (int jt = 0; jt < 2; jt++)
#pragma unroll
        for (int gq = 0; gq < 4; gq++) mr[jt][gq] = mrn[jt][gq] = make_uint2(0, 0);
    // Buffer loads: the resources end at the slice's last key, so rows past
    // it read as zero; offsets are this thread's fixed part plus a uniform
    // tile part.  Mask groups that reach past the slice are reloaded with
    // bound checks when the tail tile is computed.
    const uint32_t krow = (uint32_t)p.k_nb1 * 2u, vrow = (uint32_t)p.v_nb1 * 2u;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void *)kbase, 0, (int)(ke * krow), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void *)vbase, 0, (int)(ke * vrow), 0x00020000);
    // the mask resource is uniform (rows 0..T-1, the last one ending at the
    // slice end); this lane's row is part of its offset
    const uint32_t mrowb = (uint32_t)p.mask_nb1 * 2u;
    const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(mplane ? mplane : p.k), 0, mplane ? (int)((uint32_t)(p.T - 1) * mrowb + (uint32_t)ke * 2u) : 0, 0x00020000);
    // this lane's source offsets for the tile loads: chunk c = 64 * ii + lane
    // of wavefront load ii -> key row c / NI, piece c % NI (pieces past the
    // row's data re-read its first piece into the padding)
    const int nw = nthr >> 6;
    uint32_t koff[MKI], voff[MVI];
#pragma unroll
    for (int i = 0; i < MKI; i++) {
        const int c = 64 * (w + i * nw) + lane, r = c / NIK, pc = c % NIK;
        koff[i] = (uint32_t)r * krow + 16u * (uint32_t)(pc < D / 8 ? pc : 0);
    }
#pragma unroll
    for (int i = 0; i < MVI; i++) {
        const int c = 64 * (w + i * nw) + lane, r = c / NIV, pc = c % NIV;
        voff[i] = (uint32_t)r * vrow + 16u * (uint32_t)(pc < D / 8 ? pc : 0);
    }
    const uint32_t mth = (uint32_t)(tvalid ? t : 0) * mrowb + (uint32_t)(8 * h2);
    // tile k0n's K and V rows straight into LDS buffer `buf` (rows past the
    // slice read as zero)
    constexpr int KBUF = FA_BK * KS, VBUF = FA_BK * VSN;
    auto issue_kv = [&](int k0n, int buf) {
#pragma unroll
        for (int i = 0; i < MKI; i++) {
            const int ii = w + i * nw;
            if (ii < NIK)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (__attribute__((address_space(3))) void *)(Ks2 + buf * KBUF + 512 * ii),
                                                         16, koff[i], (uint32_t)k0n * krow, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < MVI; i++) {
            const int ii = w + i * nw;
            if (ii < NIV)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (__attribute__((address_space(3))) void *)(Vn2 + buf * VBUF + 512 * ii),
                                                         16, voff[i], (uint32_t)k0n * vrow, 0, 0);
        }
    };
    // the next tile's mask values are loaded into mrn with its K and V, at
    // the top of an iteration
    int cls_next = 1;  // class of the tile fetch_mask last prepared
    auto fetch_mask = [&](int k0n, uint2 (&mr)[2][4]) {
        cls_next = 1;
        if (mfl && k0n + FA_BK <= ke) {
            cls_next = tile_class(k0n / FA_BK);
            if (cls_next != 1) {
#pragma unroll
                for (int jt = 0; jt < 2; jt++)
#pragma unroll
                    for (int gq = 0; gq < 4; gq++) mr[jt][gq] = make_uint2(0, 0);
                return;
            }
        }
        if (mrow) {
            const uint32_t mt = (uint32_t)k0n * 2u + mth;
#pragma unroll
            for (int jt = 0; jt < 2; jt++)
#pragma unroll
                for (int gq = 0; gq < 4; gq++)
                    mr[jt][gq] = __builtin_bit_cast(
                        uint2, __builtin_amdgcn_raw_buffer_load_b64(mrs, mt + 2u * (32 * jt + 8 * gq), 0, 0));
        }
    };
    // Two LDS buffers: tile i is computed from buffer i & 1 while tile i + 1
    // lands in the other one (issued at the top of iteration i, waited for at
    // its end), so one barrier per tile separates a buffer's loads from its
    // reads and its reads from its next loads.
    if (kb < ke) {
        issue_kv(kb, 0);
        fetch_mask(kb, mr);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int k0 = kb, it = 0; k0 < ke; k0 += FA_BK, it++) {
        const int nk = min(FA_BK, ke - k0);
        const _Float16 *Ks = Ks2 + (it & 1) * KBUF;
        const _Float16 *Vn = Vn2 + (it & 1) * VBUF;
        const int cls = cls_next;  // this tile's mask class
        if (k0 + FA_BK < ke) {
            issue_kv(k0 + FA_BK, (it + 1) & 1);
            fetch_mask(k0 + FA_BK, mrn);
        }
        // a tile masked to -inf for all 32 queries adds nothing: skip its work
        if (cls != 2) {

        if (nk < FA_BK && mrow) {
            // tail tile: mask groups reaching past the range, with bound checks
#pragma unroll
            for (int jt = 0; jt < 2; jt++)
#pragma unroll
                for (int gq = 0; gq < 4; gq++) {
                    const int key = 32 * jt + 8 * gq + 4 * h2;
                    if (key + 4 > nk) {
                        uint32_t e[4];
#pragma unroll
                        for (int r = 0; r < 4; r++) e[r] = key + r < nk ? mrow[k0 + key + r] : 0u;
                        mr[jt][gq] = make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
                    }
                }
        }
        // a tile whose mask values are all zero for the whole wavefront (the
        // bulk of a causal mask) skips the per-score mask term
        uint32_t mor = 0;
#pragma unroll
        for (int jt = 0; jt < 2; jt++)
#pragma unroll
            for (int gq = 0; gq < 4; gq++) mor |= mr[jt][gq].x | mr[jt][gq].y;
        const bool mzero = __ballot(mor != 0) == 0;
        // scores of this lane: keys 32*jt + crow32(v), query t
        float s[2][16];
        // the MFMA runs (K·Qᵀ here, P·V below) issue at raised wave priority, so
        // the SIMD's other wavefront fills their gaps with its softmax work
        // (measured: 138 -> 135 us on the T = 512, S = 8192 prefill)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int jt = 0; jt < 2; jt++) {
            v16f acc;
#pragma unroll
            for (int v = 0; v < 16; v++) acc[v] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < D / 16; kk++) {
                const v8h a = *reinterpret_cast<const v8h *>(&Ks[(32 * jt + li) * KS + 16 * kk + 8 * h2]);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[kk], acc, 0, 0, 0);
            }
            if (jt == 1) __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                // relative to the reference max: x' = s2 - m_ref
                float x = fmaf(acc[v], sl2, mneg);
                if (SOFTCAP) x = p.softcap * LOG2E * tanhf(acc[v] * p.scale) + mneg;
                // mask value (0 without a mask); -inf for a masked key
                if (mzero) {
                    s[jt][v] = x;
                } else {
                    const uint32_t mw = (v & 2) ? mr[jt][v >> 2].y : mr[jt][v >> 2].x;
                    s[jt][v] = fmaf(ml2, h2f((v & 1) ? mw >> 16 : mw), x);
                }
            }
        }
        if (nk < FA_BK) {
#pragma unroll
            for (int jt = 0; jt < 2; jt++)
#pragma unroll
                for (int v = 0; v < 16; v++)
                    if (32 * jt + crow32(v, lane) >= nk) s[jt][v] = -__builtin_inff();
        }
        // Online softmax for query t (lanes l and l^32 share it) with a lazy
        // reference max: probabilities are exp2(s2 - m_ref), and m_ref moves
        // only when a score exceeds it by more than 8 (P <= 256) or on the
        // first unmasked key.  O and l are rescaled only then.
        float tmax = -__builtin_inff();
#pragma unroll
        for (int jt = 0; jt < 2; jt++)
#pragma unroll
            for (int v = 0; v < 16; v++) tmax = fmaxf(tmax, s[jt][v]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const bool need = tmax > 8.0f || (m_ref == -__builtin_inff() && tmax != -__builtin_inff());
        if (__ballot(need)) {
            if (need) {
                const float alpha = __builtin_amdgcn_exp2f(-tmax);  // o, l are 0 while m_ref is unset
                m_ref = -mneg + tmax;
                mneg = -m_ref;
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) o[dt][v] *= alpha;
#pragma unroll
                for (int jt = 0; jt < 2; jt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) s[jt][v] -= tmax;
            }
        }
        float psum = 0.0f;
#pragma unroll
        for (int jt = 0; jt < 2; jt++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float e = __builtin_amdgcn_exp2f(s[jt][v]);
                s[jt][v] = e;
                psum += e;
            }
        psum += __shfl_xor(psum, 32, 64);
        l_run += psum;
        // O^T += V^T P^T over the 64 keys: 4 MFMAs of 16 keys per d-tile
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int jt = 0; jt < 2; jt++)
#pragma unroll
            for (int m = 0; m < 2; m++) {
                v8h pb;
#pragma unroll
                for (int e = 0; e < 8; e++) pb[e] = (_Float16)s[jt][8 * m + e];
                // slot e <-> key 32*jt + 4*h2 + 8*(2m + e/4) + e%4 (matches the C layout of s)
                const int key0 = 32 * jt + 4 * h2 + 16 * m;
                // transposing reads of the key-major tile: in each 16-lane group
                // lane j gives key row key0 + j/4 at dims 4(j%4) of the group's 16
                // dims, and lane i gets keys key0 .. key0+3 of dim i
                const int lj = lane & 15, lg = (lane >> 4) & 1;
                const _Float16 *vsrc = Vn + (key0 + (lj >> 2)) * VSN + 16 * lg + 4 * (lj & 3);
#pragma unroll
                for (int dt = 0; dt < D / 32; dt++) {
                    const v4h lo = __builtin_bit_cast(v4h, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                        (__attribute__((address_space(3))) v4fp16 *)(vsrc + 32 * dt)));
                    const v4h hi = __builtin_bit_cast(v4h, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                        (__attribute__((address_space(3))) v4fp16 *)(vsrc + 8 * VSN + 32 * dt)));
                    v8h a;
#pragma unroll
                    for (int e = 0; e < 4; e++) { a[e] = lo[e]; a[4 + e] = hi[e]; }
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, o[dt], 0, 0, 0);
                }
            }
        __builtin_amdgcn_s_setprio(0);
        }  // cls != 2
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // tile it+1's K, V and mask are in
        __syncthreads();
#pragma unroll
        for (int jt = 0; jt < 2; jt++)
#pragma unroll
            for (int gq = 0; gq < 4; gq++) mr[jt][gq] = mrn[jt][gq];
    }

    // one slice: the output row, with ghip_fa_merge_rows' arithmetic for one
    // partial (weight e^(M - M) = 1 applied by the same fma, the sink, 1 / S),
    // so the bits are those of the partial-and-merge route
    if (p.direct) {
        if (tvalid) {
            const float mz = m_ref * 0.6931471805599453f, sz = l_run;
            const float M = sz != 0.0f ? mz : -__builtin_inff();
            const float wz = (sz != 0.0f && M != -__builtin_inff()) ? __expf(mz - M) : 0.0f;
            float S = sz * wz;
            float ms = 1.0f;
            if (p.sinks) {
                const float sv = p.sinks[h];
                if (sv > M) {
                    ms = __expf(M - sv);
                    S = S * ms + 1.0f;
                } else {
                    S = S + __expf(sv - M);
                }
            }
            const float sinv = S == 0.0f ? 0.0f : 1.0f / S;
            float *orow = p.dst + ((int64_t)t * p.H + h) * D;
#pragma unroll
            for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    float a = fmaf(o[dt][v], wz, 0.0f);
                    if (p.sinks && p.sinks[h] > M) a *= ms;
                    orow[32 * dt + crow32(v, lane)] = a * sinv;
                }
        }
        return;
    }
    // write this slice's partial (M in natural-log units, S, unnormalized O)
    // for query t, head h; lanes l and l^32 hold complementary d ranges
    if (tvalid) {
        float *pp = p.part + (((int64_t)t * p.H + h) * p.nsplit + z) * (2 + D);
        if (h2 == 0) {
            pp[0] = m_ref * 0.6931471805599453f;
            pp[1] = l_run;
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
            for (int v = 0; v < 16; v++) pp[2 + 32 * dt + crow32(v, lane)] = o[dt][v];
    }
}

// softcap != 0 takes its own kernel (tanh adds registers the plain body
// does not need)
template <int D, bool SOFTCAP>
__device__ __forceinline__ void fa_fwd_impl(const FaParams &p) {
    __shared__ __attribute__((aligned(16))) _Float16 Ks[2 * FA_BK * (D + FA_KPAD)];   // 2 x [key][d]
    __shared__ __attribute__((aligned(16))) _Float16 Vn[2 * FA_BK * (D + FA_VNPAD)];  // 2 x [key][d]
    fa_fwd_body<D, SOFTCAP>(p, Ks, Vn);
}

// Single-query decode over a long cache (the reference's split-KV route,
// flash_attn.rs:779-862): grid (H_kv, nsplit); a 256-thread workgroup takes
// one KV head, its G = H / H_kv query heads and one slice of the keys, and
// writes the slice's (M, S, unnormalized O) partial per head for
// ghip_fa_merge.  It is bound by reading K and V once, so it runs on the
// vector ALUs with every wavefront streaming its own quarter of the slice in
// steps of 32 keys: a step's K and V are staged into LDS and waited for, and
// the other wavefronts on the CU cover the latency (staging the next step as
// soon as a step's rows were in registers measured slower, 16.1 against
// 15.8 us at S = 8192):
//  * scores: lane pair (2j, 2j+1) holds key j's two 64-dim halves and forms
//    the G dots with v_dot2 on f16 (q is rounded to f16 as the reference
//    does, products and sums in fp32);
//  * softmax: per head, wave max / sum by DPP row operations;
//  * P V: lane l owns dims 2l, 2l+1 and reads each key's probabilities as
//    scalars (readlane).
// The four wavefronts' (M, S, O) meet in LDS at the end.
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
DEV float dpp_max_wave(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

template <int D>
__device__ __forceinline__ void fa_decode_impl(const FaParams &p) {
    constexpr int HD = D / 2;        // dims per lane of a key pair
    constexpr int NL = HD / 8;       // 16-byte K chunks per lane per key
    constexpr int RB = D * 2;        // bytes per K or V row
    constexpr int CPR = RB / 16;     // 16-byte chunks per row
    // per wavefront: this step's 32 K rows and 32 V rows, staged by direct
    // loads (chunk c of K row r at slot c ^ (r % CPR)); after the loop the
    // same bytes hold the wavefronts' partials for the combine
    __shared__ __attribute__((aligned(16))) uint8_t kv[4][2][32 * RB];
    __shared__ __attribute__((aligned(16))) _Float16 qs[8][D];
    __shared__ float wst[4][8][2];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int hk = blockIdx.x, z = blockIdx.y;
    const int G = p.H / p.H_kv;
    const int k0 = z * p.chunk, k1 = min(p.S, k0 + p.chunk);
    const int cw = (p.chunk + 3) / 4;
    const int wk0 = min(k1, k0 + w * cw), wk1 = min(k1, wk0 + cw);  // this wavefront's keys
    for (int i = tid; i < G * D; i += 256) {
        const int g = i / D, d = i - g * D;
        qs[g][d] = __builtin_bit_cast(_Float16, f2h_rn(p.q[(int64_t)(hk * G + g) * p.q_nb2 + d]));
    }
    __syncthreads();
    const uint16_t *kbase = p.k + (int64_t)hk * p.k_nb2;
    const uint16_t *vbase = p.v + (int64_t)hk * p.v_nb2;
    const int j = lane >> 1, hf = lane & 1;
    const int dl = 2 * lane;  // P V dims (D = 128); D = 64 uses lanes < 32
    const bool dv = dl < D;
    uint8_t *Ks = kv[w][0], *Vs = kv[w][1];
    float Mh[8], Sh[8], o0[8], o1[8];
#pragma unroll
    for (int g = 0; g < 8; g++) {
        Mh[g] = -__builtin_inff();
        Sh[g] = 0.0f;
        o0[g] = o1[g] = 0.0f;
    }
    // direct loads of keys kb .. kb+31 (rows past the range re-read the last
    // one); instruction i moves 64 x 16 bytes = 1024 / RB rows
    constexpr int RPI = 1024 / RB;  // rows per instruction
    auto stage = [&](int kb) {
#pragma unroll
        for (int i = 0; i < 32 / RPI; i++) {
            const int r = RPI * i + lane / CPR, slot = lane % CPR;
            const int key = min(kb + r, wk1 - 1);
            g2lds((const uint8_t *)(kbase + (int64_t)key * p.k_nb1) + 16 * (slot ^ (r % CPR)), Ks + 1024 * i);
            g2lds((const uint8_t *)(vbase + (int64_t)key * p.v_nb1) + 16 * slot, Vs + 1024 * i);
        }
    };
    for (int kb = wk0; kb < wk1; kb += 32) {
        const int nk = min(32, wk1 - kb);
        stage(kb);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();
        // scores of key kb + j for the G heads (lane half hf: dims hf*HD ..)
        uint4 kq[NL];
#pragma unroll
        for (int l = 0; l < NL; l++)
            kq[l] = *reinterpret_cast<const uint4 *>(Ks + RB * j + 16 * ((hf * NL + l) ^ (j % CPR)));
        float sg[8];
#pragma unroll
        for (int g = 0; g < 8; g++) {
            float acc = 0.0f;
            if (g < G) {
#pragma unroll
                for (int l = 0; l < NL; l++) {
                    const uint4 qv = *reinterpret_cast<const uint4 *>(&qs[g][hf * HD + 8 * l]);
                    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, kq[l].x), __builtin_bit_cast(h2v, qv.x), acc, false);
                    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, kq[l].y), __builtin_bit_cast(h2v, qv.y), acc, false);
                    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, kq[l].z), __builtin_bit_cast(h2v, qv.z), acc, false);
                    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, kq[l].w), __builtin_bit_cast(h2v, qv.w), acc, false);
                }
            }
            sg[g] = acc;
        }
        const bool live = j < nk;
        const float mk = (p.mask && live) ? h2f(p.mask[kb + j]) : 0.0f;
        // this lane's dims of the step's V rows; masked keys' rows are zeroed
        // so that they add nothing whatever the cache holds
        const uint64_t dead = __ballot(!live || mk == -__builtin_inff());
        uint32_t vq[32];
#pragma unroll
        for (int jj = 0; jj < 32; jj++) {
            const uint32_t v = dv ? *reinterpret_cast<const uint32_t *>(Vs + RB * jj + 2 * dl) : 0u;
            vq[jj] = (dead >> (2 * jj)) & 1 ? 0u : v;
        }
#pragma unroll
        for (int g = 0; g < 8; g++) {
            if (g >= G) continue;
            float x = sg[g] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sg[g]), 0xB1, 0xF, 0xF, false));
            x *= p.scale;
            if (p.softcap != 0.0f) x = p.softcap * tanhf(x);
            x += head_slope(p, hk * G + g) * mk;
            if (!live || mk == -__builtin_inff()) x = -__builtin_inff();  // masked keys are skipped outright
            const float m = dpp_max_wave(x);
            const float mn = fmaxf(Mh[g], m);
            float pj = 0.0f, alpha = 1.0f;
            if (mn != -__builtin_inff()) {
                alpha = __expf(Mh[g] - mn);  // 0 when Mh was -inf
                pj = __expf(x - mn);         // 0 for masked keys
                Mh[g] = mn;
            }
            Sh[g] = Sh[g] * alpha + 0.5f * wave_sum_dpp(pj);  // both lanes of a pair hold key j
            float a0 = o0[g] * alpha, a1 = o1[g] * alpha;
#pragma unroll
            for (int jj = 0; jj < 32; jj++) {
                const float pk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pj), 2 * jj));
                a0 = fmaf(pk, h2f(vq[jj] & 0xffff), a0);
                a1 = fmaf(pk, h2f(vq[jj] >> 16), a1);
            }
            o0[g] = a0;
            o1[g] = a1;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();  // the tile is consumed before the next step's loads land
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // ---- the four wavefronts' partials -> the workgroup's (wo aliases kv)
    float(*wo)[8][D] = reinterpret_cast<float(*)[8][D]>(&kv[0][0][0]);
    static_assert(sizeof(kv) >= sizeof(float) * 4 * 8 * D, "partials fit the K/V tiles");
    __syncthreads();  // every wavefront is done with its tile
    if (lane == 0)
        for (int g = 0; g < G; g++) {
            wst[w][g][0] = Mh[g];
            wst[w][g][1] = Sh[g];
        }
    if (dv)
        for (int g = 0; g < G; g++) {
            wo[w][g][dl] = o0[g];
            wo[w][g][dl + 1] = o1[g];
        }
    __syncthreads();
    for (int i = tid; i < G * D; i += 256) {
        const int g = i / D, d = i - g * D;
        float M = -__builtin_inff();
        for (int u = 0; u < 4; u++)
            if (wst[u][g][1] != 0.0f) M = fmaxf(M, wst[u][g][0]);
        float S = 0.0f, o = 0.0f;
        if (M != -__builtin_inff())
            for (int u = 0; u < 4; u++) {
                if (wst[u][g][1] == 0.0f) continue;
                const float e = __expf(wst[u][g][0] - M);
                S += wst[u][g][1] * e;
                o += wo[u][g][d] * e;
            }
        float *pp = p.part + ((int64_t)(hk * G + g) * p.nsplit + z) * (2 + D);
        pp[2 + d] = o;
        if (d == 0) {
            pp[0] = M;
            pp[1] = S;
        }
    }
}

// Mask tile classes for the prefill kernel: one wavefront per (plane, 32-query
// block, 64-key tile); lane l reads row 32qb + l/2, keys 64tile + 32(l&1) ..
// +31.  A tile whose values are all +-0 needs no mask loads (the scores are
// unchanged), one whose values are all -inf contributes nothing (every
// probability is 0, the running max and sums are untouched), so the forward
// kernel skips the loads, or the tile.  Rows past T count as both; tiles
// reaching past S are class 1 (the forward kernel's tail path reads those).
extern "C" __global__ void __launch_bounds__(256)
ghip_fa_mask_scan(const uint16_t *__restrict__ mask, int64_t mask_nb1, int64_t mask_nb2, int planes, int T, int S,
                  int nqb, int ntile, uint8_t *__restrict__ flags) {
    const int lane = threadIdx.x & 63;
    const int64_t id = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (id >= (int64_t)planes * nqb * ntile) return;
    const int tile = (int)(id % ntile), qb = (int)((id / ntile) % nqb), plane = (int)(id / ((int64_t)ntile * nqb));
    const int r = 32 * qb + (lane >> 1);
    bool allz = true, allinf = true;
    if (64 * tile + 64 > S) {
        allz = allinf = false;
    } else if (r < T) {
        const uint8_t *src = reinterpret_cast<const uint8_t *>(mask + (int64_t)plane * mask_nb2 + (int64_t)r * mask_nb1 +
                                                               64 * tile + 32 * (lane & 1));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 v = ld16(src + 16 * i);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                allz = allz && (w[k] & 0x7fff7fffu) == 0u;
                allinf = allinf && w[k] == 0xfc00fc00u;
            }
        }
    }
    const bool z = __ballot(!allz) == 0, ninf = __ballot(!allinf) == 0;
    if (lane == 0) flags[id] = z ? 0 : ninf ? 2 : 1;
}

// Merge the per-slice partials of one (query, head) row (reduce_partials,
// flash_attn.rs:779-835): with M = max_z M_z, the row is
// sum_z O_z e^(M_z - M) / sum_z S_z e^(M_z - M), then the sink logit joins
// the denominator.  One 256-thread workgroup per row: the slice weights are
// formed in parallel into LDS, then thread (d, part) sums slices
// part, part + P, ... of column d with independent loads, and the parts meet
// in LDS.  DV <= 256.
// Few slices per row (<= 64): WPR wavefronts per (query, head) row, 256 / WPR
// rows per workgroup; lane l owns dims l and l + 64 and lane z holds slice
// z's (M_z, S_z).  Wavefront u of a row folds slices u, u + WPR, ... in order
// with the weights exp(M_z - M) of ghip_fa_merge; the first sixteen of them are
// loaded before the weights are known, so the slice reads overlap the
// statistics.  With WPR > 1 the wavefronts' sums meet in LDS in order.
template <int WPR, int PRE = 16>
__device__ __forceinline__ void fa_merge_rows_impl(const float *__restrict__ part, const float *__restrict__ sinks,
                                                   float *__restrict__ dst, int nrows, int H, int nsplit, int DV) {
    __shared__ float red[4][2][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, u = wv % WPR;
    const int row = blockIdx.x * (4 / WPR) + wv / WPR;
    if (row >= nrows) return;  // uniform per row: all WPR wavefronts leave together
    const float *pr = part + (int64_t)row * nsplit * (2 + DV);
    const int c0 = min(lane, DV - 1), c1 = min(64 + lane, DV - 1);
    float v0[PRE], v1[PRE];
#pragma unroll
    for (int i = 0; i < PRE; i++) {
        const float *pz = pr + (int64_t)min(u + WPR * i, nsplit - 1) * (2 + DV) + 2;
        v0[i] = pz[c0];
        v1[i] = pz[c1];
    }
    float mz = -__builtin_inff(), sz = 0.0f;
    if (lane < nsplit) {
        mz = pr[(int64_t)lane * (2 + DV)];
        sz = pr[(int64_t)lane * (2 + DV) + 1];
    }
    const float M = dpp_max_wave(sz != 0.0f ? mz : -__builtin_inff());
    const float wz = (sz != 0.0f && M != -__builtin_inff()) ? __expf(mz - M) : 0.0f;
    float S = wave_sum_dpp(sz * wz);
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < PRE; i++) {
        const int z = u + WPR * i;
        if (z < nsplit) {
            const float wgt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wz), z));
            a0 = fmaf(v0[i], wgt, a0);
            a1 = fmaf(v1[i], wgt, a1);
        }
    }
#pragma unroll 4
    for (int z = u + WPR * PRE; z < nsplit; z += WPR) {
        const float *pz = pr + (int64_t)z * (2 + DV) + 2;
        const float wgt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wz), z));
        a0 = fmaf(pz[c0], wgt, a0);
        a1 = fmaf(pz[c1], wgt, a1);
    }
    if (WPR > 1) {
        red[wv][0][lane] = a0;
        red[wv][1][lane] = a1;
        __syncthreads();
        if (u != 0) return;
        a0 = 0.0f;
        a1 = 0.0f;
        for (int i = 0; i < WPR; i++) {
            a0 += red[wv + i][0][lane];
            a1 += red[wv + i][1][lane];
        }
    }
    if (sinks) {
        const float sv = sinks[row % H];
        if (sv > M) {
            const float ms = __expf(M - sv);
            a0 *= ms;
            a1 *= ms;
            S = S * ms + 1.0f;
        } else {
            S = S + __expf(sv - M);
        }
    }
    const float sinv = S == 0.0f ? 0.0f : 1.0f / S;
    if (lane < DV) dst[(int64_t)row * DV + lane] = a0 * sinv;
    if (lane + 64 < DV) dst[(int64_t)row * DV + 64 + lane] = a1 * sinv;
}

extern "C" __global__ void __launch_bounds__(256)
ghip_fa_merge_rows(const float *__restrict__ part, const float *__restrict__ sinks, float *__restrict__ dst,
                   int nrows, int H, int nsplit, int DV) {
    fa_merge_rows_impl<1>(part, sinks, dst, nrows, H, nsplit, DV);
}

// at most 4 slices (the prefill route's usual split): the first PRE = 4 loads
// are all of them (the same sums; PRE = 16 re-read the last slice 12 times)
extern "C" __global__ void __launch_bounds__(256)
ghip_fa_merge_rows_p4(const float *__restrict__ part, const float *__restrict__ sinks, float *__restrict__ dst,
                      int nrows, int H, int nsplit, int DV) {
    fa_merge_rows_impl<1, 4>(part, sinks, dst, nrows, H, nsplit, DV);
}

extern "C" __global__ void __launch_bounds__(256)
ghip_fa_merge_rows4(const float *__restrict__ part, const float *__restrict__ sinks, float *__restrict__ dst,
                    int nrows, int H, int nsplit, int DV) {
    fa_merge_rows_impl<4>(part, sinks, dst, nrows, H, nsplit, DV);
}

extern "C" __global__ void __launch_bounds__(256)
ghip_fa_merge(const float *__restrict__ part, const float *__restrict__ sinks, float *__restrict__ dst, int T,
              int H, int nsplit, int DV) {
    __shared__ float wz[1024];
    __shared__ float red[256];
    __shared__ float stat[8];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int h = row % H;
    const float *pr = part + (int64_t)row * nsplit * (2 + DV);
    // M = max over non-empty slices
    float M = -__builtin_inff();
    for (int z = tid; z < nsplit; z += 256) {
        const float *pz = pr + (int64_t)z * (2 + DV);
        if (pz[1] != 0.0f) M = fmaxf(M, pz[0]);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    if (lane == 0) stat[wv] = M;
    __syncthreads();
    M = fmaxf(fmaxf(stat[0], stat[1]), fmaxf(stat[2], stat[3]));
    const int P = 256 / DV;  // slice parts per column
    const int d = tid % DV, pt = tid / DV;
    float acc = 0.0f, S = 0.0f;
    for (int z0 = 0; z0 < nsplit; z0 += 1024) {
        const int nz = min(1024, nsplit - z0);
        __syncthreads();  // previous round's weights consumed
        for (int z = tid; z < nz; z += 256) {
            const float *pz = pr + (int64_t)(z0 + z) * (2 + DV);
            const float sz = pz[1];
            const float wgt = (sz != 0.0f && M != -__builtin_inff()) ? __expf(pz[0] - M) : 0.0f;
            wz[z] = wgt;
            S += sz * wgt;
        }
        __syncthreads();
        if (pt < P) {
#pragma unroll 8
            for (int z = pt; z < nz; z += P) acc = fmaf(pr[(int64_t)(z0 + z) * (2 + DV) + 2 + d], wz[z], acc);
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) S += __shfl_xor(S, o, 64);
    __syncthreads();
    if (lane == 0) stat[4 + wv] = S;
    red[tid] = acc;
    __syncthreads();
    if (tid < DV) {
        float o = 0.0f;
        for (int u = 0; u < P; u++) o += red[u * DV + tid];
        S = (stat[4] + stat[5]) + (stat[6] + stat[7]);
        if (sinks) {
            const float sv = sinks[h];
            if (sv > M) {
                const float ms = __expf(M - sv);
                o *= ms;
                S = S * ms + 1.0f;
            } else {
                S = S + __expf(sv - M);
            }
        }
        const float sinv = S == 0.0f ? 0.0f : 1.0f / S;
        dst[(int64_t)row * DV + tid] = o * sinv;
    }
}

// Few-row route (one query chunk, flash_attn.rs:482-703): the reference walks
// the keys of one (query, head) row in order and keeps the unnormalized V
// accumulator in f16, rounding after every rescale and every multiply-add.
// That rounding is part of the reference's result (it moves outputs by up to
// a few 1e-3 at S ~ 1000), so this route reproduces the walk: one wavefront
// per row, lane j scores key k0 + j of each 64-key tile (q rounded to f16,
// fp32 dot), then the wavefront steps through the tile's keys in order, each
// lane updating its D/64 accumulator elements with the reference's
// operations -- skip masked (-inf) keys, new max => rescale by exp(Mold - M)
// and round, then acc = f16(fma(v, vs, acc)), S = fma(S, ms, vs).
template <int D>
__device__ __forceinline__ void fa_rowseq_impl(const FaParams &p) {
    constexpr int PL = D / 64;  // accumulator elements per lane
    __shared__ float qs[4][D];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + w;  // row = t * H + h
    const bool valid = row < p.T * p.H;
    const int t = valid ? row / p.H : 0, h = valid ? row % p.H : 0;
    const int hk = h / (p.H / p.H_kv);
    const float slope = head_slope(p, h);
    const float *qr = p.q + (int64_t)h * p.q_nb2 + (int64_t)t * p.q_nb1;
    for (int d = lane; d < D; d += 64) qs[w][d] = h2f(f2h_rn(qr[d]));
    __syncthreads();
    if (!valid) return;
    const uint16_t *kbase = p.k + (int64_t)hk * p.k_nb2;
    const uint16_t *vbase = p.v + (int64_t)hk * p.v_nb2;
    float acc[PL];
#pragma unroll
    for (int i = 0; i < PL; i++) acc[i] = 0.0f;
    float M = -__builtin_inff(), S = 0.0f;
    for (int k0 = 0; k0 < p.S; k0 += 64) {
        const int key = k0 + lane;
        float s = -__builtin_inff();
        bool live = false;
        if (key < p.S) {
            const float mv = p.mask ? slope * h2f(p.mask[(int64_t)(h % p.mask_ne2) * p.mask_nb2 + (int64_t)t * p.mask_nb1 + key]) : 0.0f;
            if (mv != -__builtin_inff()) {
                live = true;
                const uint8_t *kr = (const uint8_t *)(kbase + (int64_t)key * p.k_nb1);
                float dot = 0.0f;
#pragma unroll 4
                for (int d8 = 0; d8 < D; d8 += 8) {
                    const uint4 kv = ld16(kr + 2 * d8);
                    const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        dot = fmaf(h2f(kw[e] & 0xffff), qs[w][d8 + 2 * e], dot);
                        dot = fmaf(h2f(kw[e] >> 16), qs[w][d8 + 2 * e + 1], dot);
                    }
                }
                s = dot * p.scale;
                if (p.softcap != 0.0f) s = p.softcap * tanhf(s);
                s += mv;
            }
        }
        const uint64_t livemask = __ballot(live);
        const int nk = min(64, p.S - k0);
        for (int j = 0; j < nk; j++) {
            if (!((livemask >> j) & 1)) continue;
            const float sj = __shfl(s, j, 64);
            const uint16_t *vr = vbase + (int64_t)(k0 + j) * p.v_nb1 + PL * lane;
            float vv[PL];
#pragma unroll
            for (int i = 0; i < PL; i++) vv[i] = h2f(vr[i]);
            float ms = 1.0f, vs = 1.0f;
            if (sj > M) {
                const float Mold = M;
                M = sj;
                ms = expf(Mold - M);
#pragma unroll
                for (int i = 0; i < PL; i++) acc[i] = h2f(f2h_rn(acc[i] * ms));
            } else {
                vs = expf(sj - M);
            }
#pragma unroll
            for (int i = 0; i < PL; i++) acc[i] = h2f(f2h_rn(fmaf(vv[i], vs, acc[i])));
            S = fmaf(S, ms, vs);
        }
    }
    if (p.sinks) {
        const float sh = p.sinks[h];
        float ms = 1.0f, vs = 1.0f;
        if (sh > M) {
            ms = expf(M - sh);
            M = sh;
#pragma unroll
            for (int i = 0; i < PL; i++) acc[i] *= ms;
        } else {
            vs = expf(sh - M);
        }
        S = opaque(S * ms) + vs;  // unfused, as the reference
    }
    const float sinv = S == 0.0f ? 0.0f : 1.0f / S;
    float *o = p.dst + (int64_t)row * D + PL * lane;
#pragma unroll
    for (int i = 0; i < PL; i++) o[i] = acc[i] * sinv;
}

// General shapes (any DK, DV <= 256, F32 or F16 K and V, any H / H_kv): one
// wavefront per (query, head) row walking the keys in order, as the
// reference's row walk attn_row (flash_attn.rs:482-703) -- lane j scores key
// k0 + j of each 64-key tile (q rounded to f16 for an F16 K, as
// q_to_vec_dot), then each lane updates dims lane + 64i of the accumulator
// per live key: new max => rescale by exp(Mold - M), else vs = exp(s - M);
// acc = fma(v, vs, acc).  F16ACC rounds the accumulator to f16 after every
// step (the reference's VKQ16 for an F16 V); otherwise it stays fp32 (an F32
// V, and the fp32 accumulators of the tiled and split-KV routes, which this
// kernel stands in for on shapes the other kernels do not take).
template <bool F16ACC>
__device__ __forceinline__ void fa_rowgen_impl(const FaParams &p) {
    __shared__ float qs[4][256];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + w;  // row = t * H + h
    const bool valid = row < p.T * p.H;
    const int t = valid ? row / p.H : 0, h = valid ? row % p.H : 0;
    const int hk = h / (p.H / p.H_kv);
    const int DK = p.DK, DV = p.DV;
    const float slope = head_slope(p, h);
    const float *qr = p.q + (int64_t)h * p.q_nb2 + (int64_t)t * p.q_nb1;
    for (int d = lane; d < DK; d += 64) qs[w][d] = p.k_f32 ? qr[d] : h2f(f2h_rn(qr[d]));
    __syncthreads();
    if (!valid) return;
    const uint16_t *kbase = p.k + (int64_t)hk * p.k_nb2;
    const uint16_t *vbase = p.v + (int64_t)hk * p.v_nb2;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float M = -__builtin_inff(), S = 0.0f;
    for (int k0 = 0; k0 < p.S; k0 += 64) {
        const int key = k0 + lane;
        float s = -__builtin_inff();
        bool live = false;
        if (key < p.S) {
            const float mv = p.mask ? slope * h2f(p.mask[(int64_t)(h % p.mask_ne2) * p.mask_nb2 + (int64_t)t * p.mask_nb1 + key]) : 0.0f;
            if (mv != -__builtin_inff()) {
                live = true;
                const uint16_t *kr = kbase + (int64_t)key * p.k_nb1;
                float dot = 0.0f;
                if (p.k_f32) {
                    const float *kf = reinterpret_cast<const float *>(kr);
                    for (int d = 0; d < DK; d++) dot = fmaf(kf[d], qs[w][d], dot);
                } else {
                    for (int d = 0; d < DK; d++) dot = fmaf(h2f(kr[d]), qs[w][d], dot);
                }
                s = dot * p.scale;
                if (p.softcap != 0.0f) s = p.softcap * tanhf(s);
                s += mv;
            }
        }
        const uint64_t livemask = __ballot(live);
        const int nk = min(64, p.S - k0);
        for (int j = 0; j < nk; j++) {
            if (!((livemask >> j) & 1)) continue;
            const float sj = __shfl(s, j, 64);
            const uint16_t *vr = vbase + (int64_t)(k0 + j) * p.v_nb1;
            float vv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int d = lane + 64 * i;
                vv[i] = d >= DV ? 0.0f : p.v_f32 ? reinterpret_cast<const float *>(vr)[d] : h2f(vr[d]);
            }
            float ms = 1.0f, vs = 1.0f;
            if (sj > M) {
                const float Mold = M;
                M = sj;
                ms = expf(Mold - M);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = F16ACC ? h2f(f2h_rn(acc[i] * ms)) : acc[i] * ms;
            } else {
                vs = expf(sj - M);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float a = fmaf(vv[i], vs, acc[i]);
                acc[i] = F16ACC ? h2f(f2h_rn(a)) : a;
            }
            S = fmaf(S, ms, vs);
        }
    }
    if (p.sinks) {
        const float sh = p.sinks[h];
        float ms = 1.0f, vs = 1.0f;
        if (sh > M) {
            ms = expf(M - sh);
            M = sh;
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] *= ms;
        } else {
            vs = expf(sh - M);
        }
        S = opaque(S * ms) + vs;  // unfused, as the reference
    }
    const float sinv = S == 0.0f ? 0.0f : 1.0f / S;
    float *o = p.dst + (int64_t)row * DV;
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (lane + 64 * i < DV) o[lane + 64 * i] = acc[i] * sinv;
}

extern "C" __global__ void __launch_bounds__(256) ghip_fa_rowgen_f16acc(FaParams p) { fa_rowgen_impl<true>(p); }
extern "C" __global__ void __launch_bounds__(256) ghip_fa_rowgen(FaParams p) { fa_rowgen_impl<false>(p); }

extern "C" __global__ void __launch_bounds__(512) ghip_fa_fwd_d128(FaParams p) { fa_fwd_impl<128, false>(p); }
extern "C" __global__ void __launch_bounds__(512) ghip_fa_fwd_d64(FaParams p) { fa_fwd_impl<64, false>(p); }
extern "C" __global__ void __launch_bounds__(512) ghip_fa_fwd_sc_d128(FaParams p) { fa_fwd_impl<128, true>(p); }
extern "C" __global__ void __launch_bounds__(512) ghip_fa_fwd_sc_d64(FaParams p) { fa_fwd_impl<64, true>(p); }
extern "C" __global__ void __launch_bounds__(256) ghip_fa_rowseq_d128(FaParams p) { fa_rowseq_impl<128>(p); }
extern "C" __global__ void __launch_bounds__(256) ghip_fa_rowseq_d64(FaParams p) { fa_rowseq_impl<64>(p); }
extern "C" __global__ void __launch_bounds__(256) ghip_fa_decode_d128(FaParams p) { fa_decode_impl<128>(p); }
extern "C" __global__ void __launch_bounds__(256) ghip_fa_decode_d64(FaParams p) { fa_decode_impl<64>(p); }
