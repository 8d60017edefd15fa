"""zunzuncito_amd -- MI355X-native MoE-layer hot path for the zunzuncito engines.

The product is libzzmoe.so (HIP, gfx950), whose C ABI is include/zz_gpu.h (the
engines' gpu.h, same symbols), include/zz_moe.h (the whole MoE block with
experts resident in HBM) and include/zz_gemma.h (gemma's feed-forward block and
tied embedding / lm_head around it). This module is a thin ctypes binding of that ABI for
Python callers, tests and the benchmark. There is no CPU fallback here: when the
library is missing or no gfx950 device is present, calls raise.
"""
import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libzzmoe.so")

GPU_FMT_Q40, GPU_FMT_Q80, GPU_FMT_TQ2, GPU_FMT_Q4A = 1, 2, 3, 4
ZZ_GATE_SOFTMAX_PES, ZZ_GATE_SIGMOID_BIAS, ZZ_GATE_SOFTMAX_TOPK, ZZ_GATE_DENSE = 0, 1, 2, 3
ZZ_GATE_GROUPED = 4
ZZ_ACT_GEGLU_TANH, ZZ_ACT_SWIGLU, ZZ_ACT_SWIGLU_CLAMP = 0, 1, 2

# Every symbol include/zz_gpu.h and include/zz_moe.h declare.
ABI_SYMBOLS = (
    "gpu_init", "gpu_shutdown", "gpu_ready", "gpu_name", "gpu_map", "gpu_q40_matmul",
    "gpu_matmul", "zz_moe_layer_create", "zz_moe_layer_destroy", "zz_moe_record_bytes",
    "zz_moe_expert_upload", "zz_moe_expert_upload_dev", "zz_moe_forward",
    "zz_moe_forward_dev", "zz_moe_forward_begin", "zz_moe_forward_end", "zz_moe_debug",
    "zz_moe_blockdots", "zz_moe_stats", "zz_moe_profile", "zz_moe_profile_read",
    "zz_quantize",
    "zz_last_error",
    "zz_ffn_block_create", "zz_ffn_block_destroy", "zz_ffn_block_forward_dev",
    "zz_ffn_block_forward", "zz_head_create", "zz_head_destroy", "zz_head_embed_dev",
    "zz_head_embed", "zz_head_logits_dev", "zz_head_logits", "zz_stack_create",
    "zz_stack_destroy", "zz_stack_prefill_dev", "zz_stack_decode_dev", "zz_moe_load_experts",
    "zz_gemma_stack_load", "zz_head_flash", "zz_head_use_flash", "zz_head_flash_replays",
    "zz_stack_use_flash", "zz_moe_forward_dev_noalloc", "zz_router_expf", "zz_gpu_map_refreshes", "zz_moe_dots",
)
KERNELS = ("prep", "logits", "topk", "dispatch", "ffn_up", "ffn_down", "combine", "dec_route",
           "dec_down")

_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int)
_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)


class ZzMoeDesc(C.Structure):
    _fields_ = [("D", C.c_int), ("MI", C.c_int), ("E", C.c_int), ("K", C.c_int),
                ("gating", C.c_int), ("act", C.c_int),
                ("fmt_gate", C.c_int), ("fmt_up", C.c_int), ("fmt_down", C.c_int),
                ("norm_topk", C.c_int), ("use_bias", C.c_int),
                ("eps", C.c_float), ("routed_scaling", C.c_float), ("clamp", C.c_float),
                ("n_group", C.c_int), ("topk_group", C.c_int)]


class ZzMoeWeights(C.Structure):
    _fields_ = [("router", _f32p), ("router_scale", _f32p), ("pes", _f32p), ("bias", _f32p),
                ("pre_ln", _f32p), ("post_ln", _f32p)]


class ZzMoeDump(C.Structure):
    _fields_ = [("xq", _i8p), ("xs", _f32p), ("hq", _i8p), ("hs", _f32p),
                ("uniq", _i32p), ("offs", _i32p), ("rows", _i32p), ("slots", _i32p),
                ("nu", C.c_int), ("logits", C.POINTER(C.c_double)),
                ("items", _i32p), ("items_cap", C.c_int), ("nitems", C.c_int)]


_lib = None


def lib():
    """Load libzzmoe.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `python -m zunzuncito_amd.build`")
    # torch ships its own libamdhip64.so.7 (same SONAME as /opt/rocm's): load it
    # first where torch is installed, so one HIP runtime serves both and device
    # pointers and streams can be shared with torch tensors
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(LIB_PATH)
    L.gpu_init.restype = C.c_int
    L.gpu_name.restype = C.c_char_p
    L.gpu_map.argtypes = [C.c_void_p, C.c_size_t]
    L.gpu_matmul.argtypes = [C.c_int, _f32p, _u8p, _f32p, C.c_int, C.c_int, C.c_int]
    L.gpu_q40_matmul.argtypes = [_f32p, _u8p, _f32p, C.c_int, C.c_int, C.c_int]
    L.zz_moe_layer_create.argtypes = [C.POINTER(ZzMoeDesc), C.POINTER(ZzMoeWeights)]
    L.zz_moe_layer_destroy.argtypes = [C.c_int]
    L.zz_moe_record_bytes.restype = C.c_int64
    L.zz_moe_record_bytes.argtypes = [C.POINTER(ZzMoeDesc)]
    L.zz_moe_expert_upload.argtypes = [C.c_int, C.c_int, _u8p, C.c_size_t]
    L.zz_moe_expert_upload_dev.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_size_t]
    L.zz_moe_forward.argtypes = [C.c_int, _f32p, _f32p, C.c_int, _i32p, _f32p]
    L.zz_moe_forward_dev.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                     C.c_void_p, C.c_void_p]
    L.zz_moe_forward_dev_noalloc.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                             C.c_void_p, C.c_void_p]
    L.zz_moe_forward_begin.argtypes = [C.c_int, _f32p, C.c_int]
    L.zz_moe_forward_end.argtypes = [C.c_int, _f32p, _i32p, _f32p]
    L.zz_moe_debug.argtypes = [C.c_int, C.POINTER(ZzMoeDump)]
    L.zz_moe_blockdots.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _i8p, _i32p]
    L.zz_moe_dots.argtypes = [C.c_int, _f32p, C.c_int, _i32p, _i32p]
    L.zz_moe_stats.argtypes = [C.POINTER(C.c_uint)]
    L.zz_moe_profile.argtypes = [C.c_int]
    L.zz_moe_profile_read.argtypes = [C.POINTER(C.c_double), C.POINTER(C.c_int), C.c_int]
    L.zz_router_expf.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]
    L.zz_gpu_map_refreshes.restype = C.c_longlong
    L.zz_quantize.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]
    L.zz_last_error.restype = C.c_char_p
    L.zz_ffn_block_create.argtypes = [C.c_int, C.c_int, _f32p, C.c_float]
    L.zz_ffn_block_destroy.argtypes = [C.c_int]
    L.zz_ffn_block_forward_dev.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                                           C.c_void_p]
    L.zz_ffn_block_forward.argtypes = [C.c_int, _f32p, C.c_int, _i32p, _f32p]
    L.zz_head_create.argtypes = [_u8p, C.c_int, C.c_int, _f32p, C.c_float, C.c_float, C.c_float]
    L.zz_head_destroy.argtypes = [C.c_int]
    L.zz_head_embed_dev.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
    L.zz_head_embed.argtypes = [C.c_int, _i32p, C.c_int, _f32p]
    L.zz_head_logits_dev.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                                     C.c_void_p]
    L.zz_head_logits.argtypes = [C.c_int, _f32p, C.c_int, _f32p, _i32p]
    L.zz_stack_create.argtypes = [_i32p, C.c_int, C.c_int]
    L.zz_stack_destroy.argtypes = [C.c_int]
    L.zz_stack_prefill_dev.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
    L.zz_stack_decode_dev.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p]
    L.zz_moe_load_experts.argtypes = [C.c_int, C.c_char_p, C.c_int]
    L.zz_gemma_stack_load.argtypes = [C.c_char_p, _i32p, _i32p, _i32p]
    L.zz_head_flash.argtypes = [C.c_int, _u8p, C.c_int, _i32p, C.c_int, C.c_int, _f32p, C.c_int, _i32p,
                                C.c_int]
    L.zz_head_use_flash.argtypes = [C.c_int, C.c_int]
    L.zz_head_flash_replays.argtypes = [C.POINTER(C.c_uint)]
    L.zz_stack_use_flash.argtypes = [C.c_int, C.c_int]
    _lib = L
    return L


def last_error():
    return lib().zz_last_error().decode()


def init():
    """gpu_init(); raises when no gfx950 device is usable (no silent fallback)."""
    L = lib()
    if not L.gpu_init():
        raise RuntimeError(f"gpu_init declined: {last_error()}")
    return L.gpu_name().decode()


def _p(a, t):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


def stats():
    c = (C.c_uint * 4)()
    if not lib().zz_moe_stats(c):
        raise RuntimeError(last_error())
    return list(c)


def flash_replays():
    """Rows whose FlashHead probe set a quickselect replay decided (a boundary tie)."""
    n = C.c_uint(0)
    if not lib().zz_head_flash_replays(C.byref(n)):
        raise RuntimeError(last_error())
    return n.value


def quantize_dev(fmt, d_w, d_out, n, stream=0):
    """Device f32 -> q4_0/q8_0 blocks (zz_quantize); pointers are ints."""
    if not lib().zz_quantize(fmt, C.c_void_p(d_w), C.c_void_p(d_out), n, C.c_void_p(stream or None)):
        raise RuntimeError(last_error())


def profile(on):
    if not lib().zz_moe_profile(1 if on else 0):
        raise RuntimeError(last_error())


def profile_read():
    """{kernel: (total ms, launches)} recorded since profile(True)."""
    n = len(KERNELS)
    ms = (C.c_double * n)()
    cnt = (C.c_int * n)()
    if lib().zz_moe_profile_read(ms, cnt, n) < 0:
        raise RuntimeError(last_error())
    return {k: (ms[i], cnt[i]) for i, k in enumerate(KERNELS)}


class MoeLayer:
    """One registered MoE layer (zz_moe_layer_create) with its HBM slot table."""

    def __init__(self, D, MI, E, K, gating, act, fmts, router, router_scale=None, pes=None,
                 bias=None, pre_ln=None, post_ln=None, norm_topk=1, use_bias=0, eps=1e-6,
                 routed_scaling=1.0, clamp=7.0, n_group=1, topk_group=1):
        self.desc = ZzMoeDesc(D, MI, E, K, gating, act, fmts[0], fmts[1], fmts[2], norm_topk,
                              use_bias, eps, routed_scaling, clamp, n_group, topk_group)
        keep = [np.ascontiguousarray(a, np.float32) if a is not None else None
                for a in (router, router_scale, pes, bias, pre_ln, post_ln)]
        w = ZzMoeWeights(*(_p(a, _f32p) for a in keep))
        self.D, self.MI, self.E, self.K = D, MI, E, K
        self.id = lib().zz_moe_layer_create(C.byref(self.desc), C.byref(w))
        if self.id < 0:
            raise RuntimeError(f"zz_moe_layer_create declined: {last_error()}")
        self.record_bytes = lib().zz_moe_record_bytes(C.byref(self.desc))

    def upload(self, eid, rec):
        rec = np.ascontiguousarray(rec, np.uint8)
        if not lib().zz_moe_expert_upload(self.id, eid, _p(rec, _u8p), rec.nbytes):
            raise RuntimeError(f"upload declined: {last_error()}")

    def upload_all(self, experts):
        for e in range(self.E):
            self.upload(e, experts[e * self.record_bytes:(e + 1) * self.record_bytes])

    def load_experts(self, path, li):
        """Layer li's records from a container's experts.bin (zz_moe_load_experts)."""
        if not lib().zz_moe_load_experts(self.id, os.fsencode(path), li):
            raise RuntimeError(f"zz_moe_load_experts declined: {last_error()}")

    def upload_dev(self, eid, dev_ptr, nbytes):
        if not lib().zz_moe_expert_upload_dev(self.id, eid, C.c_void_p(dev_ptr), nbytes):
            raise RuntimeError(f"upload declined: {last_error()}")

    def forward(self, x):
        """Host arrays in, (out, eidx, ewt) out; synchronous."""
        x = np.ascontiguousarray(x, np.float32)
        S = x.shape[0]
        out = np.zeros((S, self.D), np.float32)
        eidx = np.zeros(S * self.K, np.int32)
        ewt = np.zeros(S * self.K, np.float32)
        if not lib().zz_moe_forward(self.id, _p(x, _f32p), _p(out, _f32p), S, _p(eidx, _i32p),
                                    _p(ewt, _f32p)):
            raise RuntimeError(f"zz_moe_forward declined: {last_error()}")
        return out, eidx, ewt

    def forward_dev(self, d_in, d_out, S, d_eidx=0, d_ewt=0, stream=0):
        """Device pointers (ints), enqueued on `stream` (hipStream_t as int)."""
        ok = lib().zz_moe_forward_dev(self.id, C.c_void_p(d_in), C.c_void_p(d_out), S,
                                      C.c_void_p(d_eidx or None), C.c_void_p(d_ewt or None),
                                      C.c_void_p(stream or None))
        if not ok:
            raise RuntimeError(f"zz_moe_forward_dev declined: {last_error()}")

    def forward_dev_noalloc(self, d_in, d_out, S, d_eidx=0, d_ewt=0, stream=0):
        """forward_dev on the library's fixed scratch array: allocates nothing.
        Returns False (with last_error()) when the batch does not fit the scratch."""
        return bool(lib().zz_moe_forward_dev_noalloc(self.id, C.c_void_p(d_in), C.c_void_p(d_out), S,
                                                     C.c_void_p(d_eidx or None), C.c_void_p(d_ewt or None),
                                                     C.c_void_p(stream or None)))

    def debug(self, S, logits=False):
        """The last forward's dump (zz_moe_debug); logits=True adds the router
        logits [S, E] as float64 (none for gemma's decode path). items [n, 4]:
        the batched path's FFN work items (expert, union entry, first pair, pairs),
        slot i on XCD i % 8."""
        K, D, MI = self.K, self.D, self.MI
        cap = 8 * (S * K + self.E + 16)
        d = dict(xq=np.zeros((S, D), np.int8), xs=np.zeros((S, D // 32), np.float32),
                 hq=np.zeros((S * K, MI), np.int8), hs=np.zeros((S * K, MI // 32), np.float32),
                 uniq=np.zeros(self.E, np.int32), offs=np.zeros(self.E + 1, np.int32),
                 rows=np.zeros(S * K, np.int32), slots=np.zeros(S * K, np.int32))
        if logits:
            d["logits"] = np.zeros((S, self.E), np.float64)
        dump = ZzMoeDump(_p(d["xq"], _i8p), _p(d["xs"], _f32p), _p(d["hq"], _i8p),
                         _p(d["hs"], _f32p), _p(d["uniq"], _i32p), _p(d["offs"], _i32p),
                         _p(d["rows"], _i32p), _p(d["slots"], _i32p), 0,
                         _p(d["logits"], C.POINTER(C.c_double)) if logits else None)
        items = np.zeros((cap, 4), np.int32)
        dump.items, dump.items_cap = _p(items, _i32p), cap
        if not lib().zz_moe_debug(self.id, C.byref(dump)):
            raise RuntimeError(last_error())
        d["items"] = items[:min(dump.nitems, cap)]
        nu = dump.nu
        d["uniq"] = d["uniq"][:nu]
        d["offs"] = d["offs"][:nu + 1]
        return d

    def dots(self, x):
        """One forward of host rows x [S, D] on the FFN kernels' diagnostics builds
        (zz_moe_dots): their per-block int32 dots before scaling, by flat pair
        (token*K + slot): up [S*K, 2, MI, D/32] (gate, up), down [S*K, D, MI/32]."""
        x = np.ascontiguousarray(x, np.float32)
        S, K, D, MI = x.shape[0], self.K, self.D, self.MI
        up = np.zeros((S * K, 2, MI, D // 32), np.int32)
        dn = np.zeros((S * K, D, MI // 32), np.int32)
        if not lib().zz_moe_dots(self.id, _p(x, _f32p), S, _p(up, _i32p), _p(dn, _i32p)):
            raise RuntimeError(f"zz_moe_dots declined: {last_error()}")
        return up, dn

    def blockdots(self, eid, tensor, row0, nrows, xq):
        xq = np.ascontiguousarray(xq, np.int8)
        I = xq.shape[0]
        out = np.zeros((nrows, I // 32), np.int32)
        if not lib().zz_moe_blockdots(self.id, eid, tensor, row0, nrows, _p(xq, _i8p),
                                      _p(out, _i32p)):
            raise RuntimeError(last_error())
        return out

    def close(self):
        if self.id >= 0:
            lib().zz_moe_layer_destroy(self.id)
            self.id = -1


def gpu_map(arr):
    a = np.ascontiguousarray(arr)
    if not lib().gpu_map(C.c_void_p(a.ctypes.data), a.nbytes):
        raise RuntimeError(f"gpu_map declined: {last_error()}")
    return a


def gpu_matmul(fmt, W_mapped, x, O, I):
    """gpu.h matmul on a gpu_map'd weight array; returns y [S, O] or raises."""
    x = np.ascontiguousarray(x, np.float32)
    S = x.shape[0]
    y = np.zeros((S, O), np.float32)
    if not lib().gpu_matmul(fmt, _p(y, _f32p), _p(W_mapped, _u8p), _p(x, _f32p), O, I, S):
        raise RuntimeError(f"gpu_matmul declined: {last_error()}")
    return y


class FfnBlock:
    """gemma's feed-forward half of layer_fwd (zz_ffn_block_create): a MoE layer and a
    ZZ_GATE_DENSE layer of the same D, combined with post_ffn_ln and layer_scalar."""

    def __init__(self, moe, dense, post_ffn_ln, layer_scalar):
        self._post = np.ascontiguousarray(post_ffn_ln, np.float32)
        self.moe, self.dense, self.D, self.K = moe, dense, moe.D, moe.K
        self.id = lib().zz_ffn_block_create(moe.id, dense.id, _p(self._post, _f32p),
                                            float(layer_scalar))
        if self.id < 0:
            raise RuntimeError(f"zz_ffn_block_create declined: {last_error()}")

    def forward(self, H):
        """Host H [S, D] -> (new H, eidx, ewt); synchronous."""
        H = np.array(H, np.float32, order="C", copy=True)
        S = H.shape[0]
        eidx = np.zeros(S * self.K, np.int32)
        ewt = np.zeros(S * self.K, np.float32)
        if not lib().zz_ffn_block_forward(self.id, _p(H, _f32p), S, _p(eidx, _i32p), _p(ewt, _f32p)):
            raise RuntimeError(f"zz_ffn_block_forward declined: {last_error()}")
        return H, eidx, ewt

    def forward_dev(self, d_H, S, d_eidx=0, d_ewt=0, stream=0):
        if not lib().zz_ffn_block_forward_dev(self.id, C.c_void_p(d_H), S, C.c_void_p(d_eidx or None),
                                              C.c_void_p(d_ewt or None), C.c_void_p(stream or None)):
            raise RuntimeError(f"zz_ffn_block_forward_dev declined: {last_error()}")

    def close(self):
        if self.id >= 0:
            lib().zz_ffn_block_destroy(self.id)
            self.id = -1


class Head:
    """Tied q4_0 embedding / lm_head (zz_head_create)."""

    def __init__(self, table, V, D, final_norm, eps, embed_scale, softcap):
        table = np.ascontiguousarray(table, np.uint8)
        fn = np.ascontiguousarray(final_norm, np.float32)
        self.V, self.D = V, D
        self.id = lib().zz_head_create(_p(table, _u8p), V, D, _p(fn, _f32p), eps, embed_scale, softcap)
        if self.id < 0:
            raise RuntimeError(f"zz_head_create declined: {last_error()}")

    def embed(self, tok):
        tok = np.ascontiguousarray(tok, np.int32)
        H = np.zeros((tok.size, self.D), np.float32)
        if not lib().zz_head_embed(self.id, _p(tok, _i32p), tok.size, _p(H, _f32p)):
            raise RuntimeError(f"zz_head_embed declined: {last_error()}")
        return H

    def logits(self, H):
        H = np.ascontiguousarray(H, np.float32)
        S = H.shape[0]
        lg = np.zeros((S, self.V), np.float32)
        am = np.zeros(S, np.int32)
        if not lib().zz_head_logits(self.id, _p(H, _f32p), S, _p(lg, _f32p), _p(am, _i32p)):
            raise RuntimeError(f"zz_head_logits declined: {last_error()}")
        return lg, am

    def flash(self, centroids, n_clusters, token_map, cluster_size, n_probes, cluster_scale, scaled,
              force=None):
        """Attach a FlashHead (zz_head_flash): q4_0 centroids [NC, D], token_map [NC, CS]
        int32 (-1 = padding), cluster_scale [NC] f32, force ids int32."""
        cent = np.ascontiguousarray(centroids, np.uint8)
        tm = np.ascontiguousarray(token_map, np.int32)
        cs = np.ascontiguousarray(cluster_scale, np.float32)
        fo = np.ascontiguousarray(force if force is not None else np.zeros(0, np.int32), np.int32)
        if not lib().zz_head_flash(self.id, _p(cent, _u8p), n_clusters, _p(tm, _i32p), cluster_size, n_probes,
                                   _p(cs, _f32p), int(scaled), _p(fo, _i32p) if fo.size else None, fo.size):
            raise RuntimeError(f"zz_head_flash declined: {last_error()}")

    def use_flash(self, on=True):
        if not lib().zz_head_use_flash(self.id, int(bool(on))):
            raise RuntimeError(f"zz_head_use_flash declined: {last_error()}")

    def embed_dev(self, d_tok, S, d_H, stream=0):
        if not lib().zz_head_embed_dev(self.id, C.c_void_p(d_tok), S, C.c_void_p(d_H),
                                       C.c_void_p(stream or None)):
            raise RuntimeError(f"zz_head_embed_dev declined: {last_error()}")

    def logits_dev(self, d_H, S, d_logits, d_argmax=0, stream=0):
        if not lib().zz_head_logits_dev(self.id, C.c_void_p(d_H), S, C.c_void_p(d_logits),
                                        C.c_void_p(d_argmax or None), C.c_void_p(stream or None)):
            raise RuntimeError(f"zz_head_logits_dev declined: {last_error()}")

    def close(self):
        if self.id >= 0:
            lib().zz_head_destroy(self.id)
            self.id = -1


class Stack:
    """FFN blocks under a tied head (zz_stack_create): prefill and greedy decode with
    token ids kept on the device."""

    def __init__(self, blocks, head):
        ids = np.array([b.id for b in blocks], np.int32)
        self.id = lib().zz_stack_create(_p(ids, _i32p), len(ids), head.id)
        if self.id < 0:
            raise RuntimeError(f"zz_stack_create declined: {last_error()}")

    def use_flash(self, on=True):
        """The head's FlashHead on or off for this stack (zz_stack_use_flash)."""
        if not lib().zz_stack_use_flash(self.id, int(bool(on))):
            raise RuntimeError(f"zz_stack_use_flash declined: {last_error()}")

    @classmethod
    def load(cls, path):
        """A gemma4 container directory made resident (zz_gemma_stack_load)."""
        self = cls.__new__(cls)
        nl, D, V = (C.c_int(), C.c_int(), C.c_int())
        self.id = lib().zz_gemma_stack_load(os.fsencode(path), C.byref(nl), C.byref(D), C.byref(V))
        if self.id < 0:
            raise RuntimeError(f"zz_gemma_stack_load declined: {last_error()}")
        self.n_layers, self.D, self.V = nl.value, D.value, V.value
        return self

    def prefill_dev(self, d_H, S, d_tok=0, stream=0):
        if not lib().zz_stack_prefill_dev(self.id, C.c_void_p(d_H), S, C.c_void_p(d_tok or None),
                                          C.c_void_p(stream or None)):
            raise RuntimeError(f"zz_stack_prefill_dev declined: {last_error()}")

    def decode_dev(self, d_tok, n, d_logits=0, graph=False, stream=0):
        if not lib().zz_stack_decode_dev(self.id, C.c_void_p(d_tok), n, C.c_void_p(d_logits or None),
                                         1 if graph else 0, C.c_void_p(stream or None)):
            raise RuntimeError(f"zz_stack_decode_dev declined: {last_error()}")

    def close(self):
        if self.id >= 0:
            lib().zz_stack_destroy(self.id)
            self.id = -1
