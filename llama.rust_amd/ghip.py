"""ctypes binding of libghip.so (include/ghip.h) for torch-allocated device tensors.

torch supplies device memory and streams only; every computation runs in the
gfx950 kernels behind the C ABI.  There is no CPU fallback: if the library or
its code objects are missing, GhipError is raised.
"""
import ctypes as C
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libghip.so")

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, I32, MXFP4 = 0, 1, 2, 6, 8, 12, 13, 14, 15, 26, 39
Q4_1, Q5_1, Q8_1 = 3, 7, 9
Q2_K, Q3_K = 10, 11
IQ4_NL, IQ4_XS, NVFP4 = 20, 23, 40
Q1_0, Q2_0 = 41, 42
BF16 = 30
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ1_M = 16, 17, 18, 19, 21, 22, 29
OP_MUL_MAT, OP_MUL_MAT_ID, OP_FLASH_ATTN_EXT = 1, 2, 3
BLOCK = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210),
         Q8_K: (256, 292), MXFP4: (32, 17), F32: (1, 4), F16: (1, 2), I32: (1, 4),
         Q4_1: (32, 20), Q5_1: (32, 24), Q8_1: (32, 36), Q2_K: (256, 84), Q3_K: (256, 110),
         IQ4_NL: (32, 18), IQ4_XS: (256, 136), NVFP4: (64, 36), Q1_0: (128, 18), Q2_0: (64, 18), BF16: (1, 2),
         IQ2_XXS: (256, 66), IQ2_XS: (256, 74), IQ2_S: (256, 82), IQ3_XXS: (256, 98), IQ3_S: (256, 110),
         IQ1_S: (256, 50), IQ1_M: (256, 56)}
# weight type -> the activation type of its dot (vec_dot_type)
ACT_TYPE = {Q4_0: Q8_0, Q5_0: Q8_0, Q8_0: Q8_0, Q4_K: Q8_K, Q5_K: Q8_K, Q6_K: Q8_K, Q4_1: Q8_1, Q5_1: Q8_1,
            Q2_K: Q8_K, Q3_K: Q8_K, IQ4_NL: Q8_0, IQ4_XS: Q8_K, NVFP4: Q8_0, Q1_0: Q8_0, Q2_0: Q8_0, F32: F32, F16: F32, BF16: F32,
            IQ2_XXS: Q8_K, IQ2_XS: Q8_K, IQ2_S: Q8_K, IQ3_XXS: Q8_K, IQ3_S: Q8_K, IQ1_S: Q8_K, IQ1_M: Q8_K}
# int32 sub-sums per weight block (ghip_mul_mat_subsums)
SUBSUMS_PER_BLOCK = {Q4_K: 2, Q5_K: 2, Q2_K: 2, NVFP4: 4, Q1_0: 4, Q2_0: 2}


class GhipError(RuntimeError):
    pass


class Tensor(C.Structure):
    _fields_ = [("type", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_uint64 * 4),
                ("data", C.c_void_p), ("op_params", C.c_int32 * 16)]


class GNode(C.Structure):
    """struct ghip_node"""
    _fields_ = [("op", C.c_int32), ("src", C.POINTER(Tensor) * 5), ("dst", C.POINTER(Tensor))]


class Node:
    """One graph node for Backend.graph_compute: the op and ggml views of its
    sources and destination (kept alive with the node)."""

    def __init__(self, op, srcs, dst):
        self.op, self.srcs, self.dst = op, list(srcs), dst


def mul_mat_node(w, wtype, k, x, out):
    xty = F32 if x.dtype == torch.float32 else ACT_TYPE[wtype]
    return Node(OP_MUL_MAT, [describe(w, wtype, k), describe(x, xty, k)], describe(out, F32))


def mul_mat_id_node(experts, k, b, ids, out, ty=None):
    ty = MXFP4 if ty is None else ty
    return Node(OP_MUL_MAT_ID, [describe(experts, ty, k), describe(b, F32), describe(ids, I32)], describe(out, F32))


def flash_attn_node(q, k, v, mask, sinks, out, scale=1.0, max_bias=0.0, softcap=0.0):
    import struct
    d = describe(out, F32)
    for i, f in enumerate((scale, max_bias, softcap)):
        d.op_params[i] = struct.unpack("<i", struct.pack("<f", f))[0]
    kvt = lambda t: F32 if t.dtype == torch.float32 else F16
    return Node(OP_FLASH_ATTN_EXT, [describe(q, F32), describe(k, kvt(k)), describe(v, kvt(v)), describe(mask, F16),
                                    describe(sinks, F32)], d)


def row_size(ty, n):
    qk, sz = BLOCK[ty]
    if n % qk:
        raise ValueError(f"row length {n} not a multiple of block size {qk}")
    return n // qk * sz


def describe(t, ty, ne0=None):
    """ggml view of a torch tensor.  For quantized types `t` is uint8 with the
    packed rows in its last dim and ne0 gives the logical row length."""
    d = Tensor()
    d.type = ty
    if t is None:
        return None
    if ty in (F32, F16, BF16, I32):
        shape = list(t.shape)[::-1] + [1] * (4 - t.dim())
        nb = [s * t.element_size() for s in t.stride()][::-1]
        ne = shape[:4]
    else:
        assert t.dtype == torch.uint8
        rows_shape = list(t.shape[:-1])[::-1]
        ne = [ne0] + rows_shape + [1] * (3 - len(rows_shape))
        nb = [BLOCK[ty][1]] + [s for s in t.stride()[:-1]][::-1]
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1])
    for i in range(4):
        d.ne[i] = int(ne[i])
        d.nb[i] = int(nb[i])
    d.data = t.data_ptr()
    return d


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise GhipError(f"{LIB_PATH} is not built: run llama.rust_amd/build.py")
        L = C.CDLL(LIB_PATH)
        P = C.POINTER(Tensor)
        L.ghip_init.restype = C.c_int
        L.ghip_init.argtypes = [C.c_int, C.POINTER(C.c_void_p)]
        L.ghip_free.restype = None
        L.ghip_free.argtypes = [C.c_void_p]
        L.ghip_last_error.restype = C.c_char_p
        L.ghip_last_error.argtypes = [C.c_void_p]
        L.ghip_synchronize.restype = C.c_int
        L.ghip_synchronize.argtypes = [C.c_void_p, C.c_void_p]
        L.ghip_supports_op.restype = C.c_int
        L.ghip_supports_op.argtypes = [C.c_int, P, C.POINTER(P), C.c_int]
        L.ghip_mul_mat.restype = C.c_int
        L.ghip_mul_mat.argtypes = [C.c_void_p, P, P, P, C.c_void_p]
        L.ghip_mul_mat_subsums.restype = C.c_int
        L.ghip_mul_mat_subsums.argtypes = [C.c_void_p, P, P, C.c_void_p, C.c_void_p]
        L.ghip_mul_mat_act.restype = C.c_int
        L.ghip_mul_mat_act.argtypes = [C.c_void_p, P, P, C.c_void_p, C.c_void_p]
        L.ghip_quantize_chunk.restype = C.c_int
        L.ghip_quantize_chunk.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64,
                                          C.c_void_p]
        L.ghip_mul_mat_id.restype = C.c_int
        L.ghip_mul_mat_id.argtypes = [C.c_void_p, P, P, P, P, C.c_void_p]
        L.ghip_mul_mat_id_subsums.restype = C.c_int
        L.ghip_mul_mat_id_subsums.argtypes = [C.c_void_p, P, P, P, C.c_void_p, C.c_void_p]
        L.ghip_graph_compute.restype = C.c_int
        L.ghip_graph_compute.argtypes = [C.c_void_p, C.POINTER(GNode), C.c_int32, C.c_void_p]
        L.ghip_set_workspace.restype = C.c_int
        L.ghip_set_workspace.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        L.ghip_workspace_size.restype = C.c_int
        L.ghip_workspace_size.argtypes = [C.c_int, P, C.POINTER(P), C.c_int, C.POINTER(C.c_size_t)]
        L.ghip_weight_register.restype = C.c_int
        L.ghip_weight_register.argtypes = [C.c_void_p, P, C.c_void_p]
        L.ghip_weight_unregister.restype = C.c_int
        L.ghip_weight_unregister.argtypes = [C.c_void_p, P]
        L.ghip_weight_cache_stats.restype = C.c_int
        L.ghip_weight_cache_stats.argtypes = [C.c_void_p] + [C.POINTER(C.c_size_t)] * 3
        L.ghip_flash_attn_ext.restype = C.c_int
        L.ghip_flash_attn_ext.argtypes = [C.c_void_p, P, P, P, P, P, P, C.c_void_p]
        _lib = L
    return _lib


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


class Backend:
    """One ghip context on one device (BackendI of the reference)."""

    def __init__(self, device=0):
        self.device = device
        self._ctx = C.c_void_p()
        st = lib().ghip_init(device, C.byref(self._ctx))
        if st != 0:
            raise GhipError(f"ghip_init({device}) failed with status {st}")

    def close(self):
        if self._ctx:
            lib().ghip_free(self._ctx)
            self._ctx = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st, what):
        if st != 0:
            msg = lib().ghip_last_error(self._ctx).decode()
            raise GhipError(f"{what}: status {st}: {msg}")

    # ---- MUL_MAT
    def mul_mat(self, w, wtype, k, x, out=None):
        """out[M, N] = x[M, K] @ dequant(w[N, row_bytes]).T"""
        n, m = w.shape[0], x.shape[0]
        if out is None:
            out = torch.empty((m, n), dtype=torch.float32, device=x.device)
        xty = F32 if x.dtype == torch.float32 else ACT_TYPE[wtype]
        a, b, d = describe(w, wtype, k), describe(x, xty, k), describe(out, F32)
        self._check(lib().ghip_mul_mat(self._ctx, C.byref(a), C.byref(b), C.byref(d), _stream()), "ghip_mul_mat")
        return out

    def mul_mat_subsums(self, w, wtype, k, x):
        n, m = w.shape[0], x.shape[0]
        nb = k // BLOCK[wtype][0]
        per = SUBSUMS_PER_BLOCK.get(wtype, 1) * nb
        sub = torch.empty((m, n, per), dtype=torch.int32, device=x.device)
        a, b = describe(w, wtype, k), describe(x, F32)
        self._check(lib().ghip_mul_mat_subsums(self._ctx, C.byref(a), C.byref(b), C.c_void_p(sub.data_ptr()),
                                               _stream()), "ghip_mul_mat_subsums")
        if wtype in (Q4_K, Q5_K, Q2_K):
            sub = sub.view(m, n, nb, 2)
        return sub

    def mul_mat_act(self, w, wtype, k, x):
        m = x.shape[0]
        act_ty = ACT_TYPE[wtype]
        out = torch.empty((m, row_size(act_ty, k)), dtype=torch.uint8, device=x.device)
        a, b = describe(w, wtype, k), describe(x, F32)
        self._check(lib().ghip_mul_mat_act(self._ctx, C.byref(a), C.byref(b), C.c_void_p(out.data_ptr()),
                                           _stream()), "ghip_mul_mat_act")
        return out

    def supports_mul_mat(self, w, wtype, k, x, out):
        a, b, d = describe(w, wtype, k), describe(x, F32), describe(out, F32)
        srcs = (C.POINTER(Tensor) * 2)(C.pointer(a), C.pointer(b))
        return bool(lib().ghip_supports_op(OP_MUL_MAT, C.byref(d), srcs, 2))

    # ---- weight cache
    def register_weight(self, w, wtype, k):
        """Keep the kernels' device layouts of weight w (immutable from now on)."""
        a = describe(w, wtype, k)
        self._check(lib().ghip_weight_register(self._ctx, C.byref(a), _stream()), "ghip_weight_register")

    def unregister_weight(self, w, wtype, k):
        a = describe(w, wtype, k)
        self._check(lib().ghip_weight_unregister(self._ctx, C.byref(a)), "ghip_weight_unregister")

    def weight_cache_stats(self):
        """(weights kept, bytes kept, copies built so far)"""
        v = [C.c_size_t() for _ in range(3)]
        self._check(lib().ghip_weight_cache_stats(self._ctx, *[C.byref(x) for x in v]), "ghip_weight_cache_stats")
        return tuple(x.value for x in v)

    def quantize(self, x, ty):
        """GGUF blocks of `ty` for the f32 rows of x [rows, n] (ggml_quantize_chunk)."""
        x = x.contiguous()
        n = x.shape[-1]
        rows = x.numel() // n
        out = torch.empty((rows, row_size(ty, n)), dtype=torch.uint8, device=x.device)
        self._check(lib().ghip_quantize_chunk(self._ctx, ty, C.c_void_p(x.data_ptr()), C.c_void_p(out.data_ptr()),
                                              rows, n, _stream()), "ghip_quantize_chunk")
        return out

    # ---- MUL_MAT_ID
    def mul_mat_id(self, experts, k, b, ids, out=None, ty=None):
        """experts [n_as, rows, row_bytes] (MXFP4 unless ty names another
        type), b [n_tokens, ne11, K] f32, ids [n_tokens, n_ids] int32 ->
        out [n_tokens, n_ids, rows] f32."""
        ty = MXFP4 if ty is None else ty
        n_tokens, n_ids = ids.shape
        if out is None:
            out = torch.empty((n_tokens, n_ids, experts.shape[1]), dtype=torch.float32, device=b.device)
        a, tb, ti, d = describe(experts, ty, k), describe(b, F32), describe(ids, I32), describe(out, F32)
        self._check(lib().ghip_mul_mat_id(self._ctx, C.byref(a), C.byref(tb), C.byref(ti), C.byref(d), _stream()),
                    "ghip_mul_mat_id")
        return out

    def mul_mat_id_subsums(self, experts, k, b, ids, ty=None):
        """MXFP4: the int32 block dots [n_tokens, n_ids, rows, K / 32];
        Q4_K / Q5_K: (iacc, imin) per super-block [.., rows, K / 256, 2];
        Q6_K: is per super-block [.., rows, K / 256]."""
        ty = MXFP4 if ty is None else ty
        n_tokens, n_ids = ids.shape
        per = {MXFP4: (k // 32,), Q4_K: (k // 256, 2), Q5_K: (k // 256, 2), Q6_K: (k // 256,)}.get(ty)
        if per is None:  # the further types: their MUL_MAT sub-sum row (ghip_mul_mat_subsums)
            per = (k // BLOCK[ty][0] * SUBSUMS_PER_BLOCK.get(ty, 1),)
        sub = torch.full((n_tokens, n_ids, experts.shape[1], *per), -1, dtype=torch.int32, device=b.device)
        a, tb, ti = describe(experts, ty, k), describe(b, F32), describe(ids, I32)
        self._check(lib().ghip_mul_mat_id_subsums(self._ctx, C.byref(a), C.byref(tb), C.byref(ti),
                                                  C.c_void_p(sub.data_ptr()), _stream()), "ghip_mul_mat_id_subsums")
        return sub

    # ---- FLASH_ATTN_EXT
    def flash_attn_ext(self, q, k, v, mask=None, sinks=None, scale=1.0, max_bias=0.0, softcap=0.0, out=None):
        """q [(n_seq,) H, T, DK] f32, k [(n_seq,) H_kv, S, DK] / v [(n_seq,) H_kv, S, DV] f16 or
        f32, mask [(m3, m2,) T, S] f16 (planes broadcast to heads by h % m2 and to
        sequences by i3 % m3), sinks [H] f32 -> [(n_seq,) T, H, DV] f32."""
        import struct
        H, T = q.shape[-3], q.shape[-2]
        if out is None:
            out = torch.empty(tuple(q.shape[:-3]) + (T, H, v.shape[-1]), dtype=torch.float32, device=q.device)
        kvt = lambda t: F32 if t.dtype == torch.float32 else F16
        tq, tk, tv = describe(q, F32), describe(k, kvt(k)), describe(v, kvt(v))
        tm, ts, td = describe(mask, F16), describe(sinks, F32), describe(out, F32)
        for i, f in enumerate((scale, max_bias, softcap)):
            td.op_params[i] = struct.unpack("<i", struct.pack("<f", f))[0]
        ref = lambda t: C.byref(t) if t is not None else None
        self._check(lib().ghip_flash_attn_ext(self._ctx, ref(tq), ref(tk), ref(tv), ref(tm), ref(ts), ref(td),
                                              _stream()), "ghip_flash_attn_ext")
        return out

    # ---- graph
    def graph_compute(self, nodes):
        """ghip_graph_compute over a list of Node (mul_mat_node, ...), in order."""
        arr = (GNode * max(1, len(nodes)))()
        for i, nd in enumerate(nodes):
            arr[i].op = nd.op
            for j, t in enumerate(nd.srcs[:5]):
                arr[i].src[j] = C.pointer(t) if t is not None else None
            arr[i].dst = C.pointer(nd.dst) if nd.dst is not None else None
        self._check(lib().ghip_graph_compute(self._ctx, arr, len(nodes), _stream()), "ghip_graph_compute")

    # ---- workspace
    def set_workspace(self, buf):
        """Use the device tensor `buf` (kept alive here) as the context's
        workspace; None returns to the library-owned one."""
        self._ws = buf
        ptr, n = (buf.data_ptr(), buf.numel() * buf.element_size()) if buf is not None else (None, 0)
        self._check(lib().ghip_set_workspace(self._ctx, ptr, n), "ghip_set_workspace")

    @staticmethod
    def workspace_size(node):
        """Workspace bytes of one graph node (ghip_workspace_size)."""
        P = C.POINTER(Tensor)
        srcs = (P * 5)(*[C.pointer(t) if t is not None else None for t in (node.srcs + [None] * 5)[:5]])
        out = C.c_size_t(0)
        st = lib().ghip_workspace_size(node.op, C.pointer(node.dst), srcs, len(node.srcs), C.byref(out))
        if st != 0:
            raise GhipError(f"ghip_workspace_size: status {st}")
        return out.value

    def synchronize(self):
        self._check(lib().ghip_synchronize(self._ctx, _stream()), "ghip_synchronize")


# ---------------------------------------------------------------- GGUF files
class GgufTensorInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("type", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_uint64 * 4),
                ("offset", C.c_uint64), ("size", C.c_uint64), ("part", C.c_int32)]


def _gguf_lib():
    L = lib()
    if not getattr(L, "_gguf_ready", False):
        V, P = C.c_void_p, C.POINTER
        sig = {
            "ghip_gguf_open": (C.c_int, [C.c_char_p, C.c_int, P(V), C.c_char_p, C.c_size_t]),
            "ghip_gguf_close": (None, [V]),
            "ghip_gguf_version": (C.c_uint32, [V]), "ghip_gguf_alignment": (C.c_uint64, [V]),
            "ghip_gguf_data_offset": (C.c_uint64, [V]), "ghip_gguf_n_parts": (C.c_int64, [V]),
            "ghip_gguf_n_kv": (C.c_int64, [V]), "ghip_gguf_key": (C.c_char_p, [V, C.c_int64]),
            "ghip_gguf_find_key": (C.c_int64, [V, C.c_char_p]), "ghip_gguf_kv_type": (C.c_int32, [V, C.c_int64]),
            "ghip_gguf_arr_type": (C.c_int32, [V, C.c_int64]), "ghip_gguf_arr_n": (C.c_int64, [V, C.c_int64]),
            "ghip_gguf_get_u32": (C.c_int, [V, C.c_int64, C.c_int64, P(C.c_uint32)]),
            "ghip_gguf_get_u16": (C.c_int, [V, C.c_int64, C.c_int64, P(C.c_uint16)]),
            "ghip_gguf_get_f32": (C.c_int, [V, C.c_int64, C.c_int64, P(C.c_float)]),
            "ghip_gguf_get_i64": (C.c_int, [V, C.c_int64, C.c_int64, P(C.c_int64)]),
            "ghip_gguf_get_f64": (C.c_int, [V, C.c_int64, C.c_int64, P(C.c_double)]),
            "ghip_gguf_get_bool": (C.c_int, [V, C.c_int64, C.c_int64, P(C.c_int)]),
            "ghip_gguf_get_str": (C.c_int, [V, C.c_int64, C.c_int64, P(C.c_void_p), P(C.c_size_t)]),
            "ghip_gguf_n_tensors": (C.c_int64, [V]), "ghip_gguf_find_tensor": (C.c_int64, [V, C.c_char_p]),
            "ghip_gguf_tensor": (C.c_int, [V, C.c_int64, P(GgufTensorInfo)]),
            "ghip_gguf_tensor_data": (C.c_void_p, [V, C.c_int64]),
            "ghip_gguf_upload": (C.c_int, [V, V, C.c_int64, V, C.c_int, V]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        L._gguf_ready = True
    return L


class Gguf:
    """A GGUF file opened by the library's reader (ghip_gguf_open)."""

    def __init__(self, path, follow_splits=True):
        L = _gguf_lib()
        self._g = C.c_void_p()
        err = C.create_string_buffer(512)
        if L.ghip_gguf_open(os.fsencode(path), int(follow_splits), C.byref(self._g), err, 512) != 0:
            raise GhipError(err.value.decode())

    def close(self):
        if self._g:
            _gguf_lib().ghip_gguf_close(self._g)
            self._g = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def version(self):
        return _gguf_lib().ghip_gguf_version(self._g)

    @property
    def alignment(self):
        return _gguf_lib().ghip_gguf_alignment(self._g)

    @property
    def data_offset(self):
        return _gguf_lib().ghip_gguf_data_offset(self._g)

    @property
    def n_parts(self):
        return _gguf_lib().ghip_gguf_n_parts(self._g)

    def keys(self):
        L = _gguf_lib()
        return [L.ghip_gguf_key(self._g, i).decode() for i in range(L.ghip_gguf_n_kv(self._g))]

    def kv_type(self, key):
        L = _gguf_lib()
        return L.ghip_gguf_kv_type(self._g, L.ghip_gguf_find_key(self._g, key.encode()))

    def _scalar(self, i, j):
        """Python value of kv i (j = -1) or array element j, by its stored type."""
        L = _gguf_lib()
        ty = L.ghip_gguf_kv_type(self._g, i) if j < 0 else L.ghip_gguf_arr_type(self._g, i)
        if ty == GGUF_STRING:
            p, n = C.c_void_p(), C.c_size_t()
            L.ghip_gguf_get_str(self._g, i, j, C.byref(p), C.byref(n))
            return C.string_at(p, n.value).decode("utf-8", errors="surrogateescape")
        if ty == GGUF_BOOL:
            b = C.c_int()
            L.ghip_gguf_get_bool(self._g, i, j, C.byref(b))
            return bool(b.value)
        if ty in (GGUF_FLOAT32, GGUF_FLOAT64):
            f = C.c_double()
            L.ghip_gguf_get_f64(self._g, i, j, C.byref(f))
            return f.value
        v = C.c_int64()
        L.ghip_gguf_get_i64(self._g, i, j, C.byref(v))
        return v.value

    def get(self, key, default=None):
        """The value of `key` (arrays as Python lists), default if absent."""
        L = _gguf_lib()
        i = L.ghip_gguf_find_key(self._g, key.encode())
        if i < 0:
            return default
        if L.ghip_gguf_kv_type(self._g, i) == GGUF_ARRAY:
            return [self._scalar(i, j) for j in range(L.ghip_gguf_arr_n(self._g, i))]
        return self._scalar(i, -1)

    def get_u32(self, key):
        """Value::as_u32 semantics (None when it does not apply)."""
        L = _gguf_lib()
        out = C.c_uint32()
        ok = L.ghip_gguf_get_u32(self._g, L.ghip_gguf_find_key(self._g, key.encode()), -1, C.byref(out))
        return out.value if ok else None

    def get_f32(self, key):
        L = _gguf_lib()
        out = C.c_float()
        ok = L.ghip_gguf_get_f32(self._g, L.ghip_gguf_find_key(self._g, key.encode()), -1, C.byref(out))
        return out.value if ok else None

    def tensors(self):
        L = _gguf_lib()
        out = []
        for i in range(L.ghip_gguf_n_tensors(self._g)):
            t = GgufTensorInfo()
            L.ghip_gguf_tensor(self._g, i, C.byref(t))
            out.append({"name": t.name.decode(), "type": t.type, "ne": list(t.ne), "nb": list(t.nb),
                        "offset": t.offset, "size": t.size, "part": t.part})
        return out

    def tensor_bytes(self, name):
        """A copy of the tensor's bytes as stored in the file."""
        L = _gguf_lib()
        i = L.ghip_gguf_find_tensor(self._g, name.encode())
        t = GgufTensorInfo()
        if i < 0 or L.ghip_gguf_tensor(self._g, i, C.byref(t)) != 0:
            raise KeyError(name)
        p = L.ghip_gguf_tensor_data(self._g, i)
        if not p:
            raise GhipError(f"tensor {name}: bytes outside the file")
        return C.string_at(p, t.size)

    def upload(self, be, name, register=False):
        """The tensor on the device as a uint8 tensor [rows..., row_bytes]
        (ghip_gguf_upload), optionally registered with `be`."""
        L = _gguf_lib()
        i = L.ghip_gguf_find_tensor(self._g, name.encode())
        t = GgufTensorInfo()
        if i < 0 or L.ghip_gguf_tensor(self._g, i, C.byref(t)) != 0:
            raise KeyError(name)
        shape = [int(t.ne[3]), int(t.ne[2]), int(t.ne[1])]
        while len(shape) > 1 and shape[0] == 1:
            shape.pop(0)
        dev = torch.empty(shape + [int(t.nb[1])], dtype=torch.uint8, device="cuda")
        be._check(L.ghip_gguf_upload(be._ctx, self._g, i, C.c_void_p(dev.data_ptr()), int(register), _stream()),
                  "ghip_gguf_upload")
        return dev


GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32 = range(7)
GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64 = range(7, 13)
