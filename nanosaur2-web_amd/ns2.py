"""ctypes binding of the ns2 C ABI (include/ns2.h) for Python callers (tests, bench).

Device buffers are passed as integer addresses (e.g. ``tensor.data_ptr()`` of a HIP tensor);
every call checks the status code and raises NS2Error with the library's message. The library
must have been built (``make -C nanosaur2-web_amd``); importing this module never falls back
to anything else.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libns2.so")
ADDON_PATH = os.path.join(HERE, "lib", "ns2.node")

ACT = {"none": 0, "silu": 1, "gelu_tanh": 2}
EW = {"add": 0, "sub": 1, "silu": 2, "copy": 3}

c_int, c_ll, c_float, c_size, c_vp = ctypes.c_int, ctypes.c_longlong, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p

# name -> argtypes (all return int status unless listed in _RESTYPES)
SIGNATURES = {
    "ns2_init": [c_int],
    "ns2_last_error": [],
    "ns2_device_info": [ctypes.c_char_p, c_size, ctypes.POINTER(c_int), ctypes.POINTER(c_size)],
    "ns2_set_stream": [c_vp],
    "ns2_get_stream": [],
    "ns2_malloc": [ctypes.POINTER(c_vp), c_size],
    "ns2_free": [c_vp],
    "ns2_pool_round": [c_size],
    "ns2_pool_get": [c_size, ctypes.POINTER(c_vp), ctypes.POINTER(c_size)],
    "ns2_pool_put": [c_vp, c_size],
    "ns2_pool_trim": [],
    "ns2_pool_stats": [ctypes.POINTER(c_size), ctypes.POINTER(c_size)],
    "ns2_h2d": [c_vp, c_vp, c_size],
    "ns2_d2h": [c_vp, c_vp, c_size],
    "ns2_sync": [],
    "ns2_fill_u32": [c_vp, ctypes.c_uint32, c_size],
    "ns2_graph_begin": [],
    "ns2_graph_end": [ctypes.POINTER(c_vp)],
    "ns2_graph_launch": [c_vp],
    "ns2_graph_destroy": [c_vp],
    "ns2_event_create": [ctypes.POINTER(c_vp)],
    "ns2_event_record": [c_vp],
    "ns2_event_elapsed": [c_vp, c_vp, ctypes.POINTER(c_float)],
    "ns2_event_destroy": [c_vp],
    "ns2_profile_enable": [c_int],
    "ns2_profile_reset": [],
    "ns2_profile_report": [ctypes.c_char_p, c_size],
    "ns2_hadamard256": [c_vp, c_vp, c_ll],
    "ns2_rotate_f16": [c_vp, c_int, c_vp, c_int, c_int, c_int, c_int],
    "ns2_linear_i8_tiled": [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll, c_float,
                            c_int, c_int, c_vp, c_ll],
    "ns2_linear_i8_tiled_lora": [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll, c_float,
                            c_int, c_int, c_vp, c_ll, c_vp, c_vp, c_int],
    "ns2_tile_i8_weight": [c_vp, c_vp, c_int, c_int],
    "ns2_tile_i8_weight_glu": [c_vp, c_vp, c_int, c_int],
    "ns2_linear_i8_glu_rot_tiled": [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_float, c_int],
    "ns2_linear_i8_glu_rot_tiled_lora": [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_float, c_int, c_vp, c_vp, c_int],
    "ns2_linear_i8": [c_vp, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int,
                      c_ll, c_float, c_int, c_int, c_vp, c_ll],
    "ns2_linear_i8_lora": [c_vp, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int,
                      c_ll, c_float, c_int, c_int, c_vp, c_ll, c_vp, c_vp, c_int],
    "ns2_linear_bf16": [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll,
                        c_float, c_int, c_int, c_vp, c_ll],
    "ns2_linear_bf16_lora": [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll,
                        c_float, c_int, c_int, c_vp, c_ll, c_vp, c_vp, c_int],
    "ns2_tile_bf16_weight": [c_vp, c_vp, c_int, c_int],
    "ns2_linear_f16w_tiled": [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll, c_float, c_int, c_int,
                              c_vp, c_ll],
    "ns2_linear_f16w_tiled_lora": [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll, c_float, c_int, c_int,
                                   c_vp, c_ll, c_vp, c_vp, c_int],
    "ns2_norm_mod_f16": [c_vp, c_vp, c_ll, c_ll, c_int, c_int, c_vp, c_float, c_vp, c_int],
    "ns2_to_tiled_f16": [c_vp, c_int, c_vp, c_int, c_vp, c_int, c_int],
    "ns2_attention": [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                      c_int, c_ll, c_ll, c_ll, c_ll, c_ll, c_ll, c_ll, c_ll, c_float, c_vp, c_int,
                      c_ll, c_vp, c_vp, c_float, c_vp, c_ll, c_int],
    "ns2_attention_noalloc": [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                              c_int, c_ll, c_ll, c_ll, c_ll, c_ll, c_ll, c_ll, c_ll, c_float, c_vp, c_int,
                              c_ll, c_vp, c_vp, c_float, c_vp, c_ll, c_int],
    "ns2_attention_text": [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                           c_ll, c_ll, c_ll, c_ll, c_float, c_vp, c_int, c_vp, c_vp, c_float, c_vp, c_ll, c_int,
                           c_vp, c_vp, c_int, c_int],
    "ns2_attention_vpacked": [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                              c_ll, c_ll, c_ll, c_ll, c_float, c_vp, c_int, c_vp, c_vp, c_float, c_vp, c_ll, c_int,
                              c_vp, c_vp, c_int, c_int, c_vp, c_int],
    "ns2_attention_vpack_bytes": [c_int, c_int, c_int],
    "ns2_linear_i8_tiled_vpack": [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll, c_float, c_int,
                                  c_vp, c_vp, c_int, c_vp, c_int, c_int, c_int, c_int],
    "ns2_attention_rows": [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                           c_ll, c_ll, c_ll, c_int, c_int],
    "ns2_attention_rows_f16kv": [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                 c_ll, c_ll, c_ll, c_int, c_int],
    "ns2_attention_rows_f16kv_oproj": [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int,
                                       c_int, c_ll, c_ll, c_ll, c_int, c_int, c_int],
    "ns2_parts_add_rmsnorm": [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_float],
    "ns2_parts_add_rmsnorm_tiled": [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_float],
    "ns2_linear_f16w_tiled_head_norm_f16kv": [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp, c_int, c_vp, c_int,
                                              c_int, c_vp, c_ll, c_int, c_float, c_vp, c_int],
    "ns2_linear_f16w_tiled_glu_down": [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp, c_int, c_vp],
    "ns2_head_norm": [c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll, c_ll, c_vp, c_ll, c_float],
    "ns2_head_norm2": [c_vp, c_vp, c_int, c_vp, c_int, c_int, c_int, c_int, c_ll, c_ll, c_vp, c_ll, c_float],
    "ns2_norm_mod": [c_vp, c_vp, c_ll, c_ll, c_int, c_int, c_vp, c_float, c_vp],
    "ns2_norm_mod_rotate_f16": [c_vp, c_vp, c_ll, c_ll, c_int, c_int, c_vp, c_float, c_vp, c_int],
    "ns2_glu": [c_vp, c_vp, c_int, c_int, c_int],
    "ns2_glu_rotate_f16": [c_vp, c_vp, c_int, c_int, c_int, c_int],
    "ns2_elementwise": [c_int, c_vp, c_vp, c_vp, c_ll],
    "ns2_accumulate": [c_vp, c_vp, c_ll],
    "ns2_add_rows": [c_vp, c_vp, c_vp, c_int, c_int],
    "ns2_row_sum": [c_vp, c_vp, c_vp, c_int, c_int, c_float],
    "ns2_rmsnorm": [c_vp, c_vp, c_vp, c_int, c_int, c_float],
    "ns2_add_rmsnorm": [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_float],
    "ns2_transpose": [c_vp, c_vp, c_int, c_int],
    "ns2_linear_bf16_glu": [c_vp, c_int, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int],
    "ns2_linear_bf16_glu_down": [c_vp, c_int, c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp, c_int, c_vp],
    "ns2_linear_bf16_head_norm": [c_vp, c_int, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp, c_int, c_vp, c_int,
                                  c_int, c_vp, c_ll, c_int, c_float],
    "ns2_linear_bf16_head_norm_f16kv": [c_vp, c_int, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp, c_int, c_vp,
                                        c_int, c_int, c_vp, c_ll, c_int, c_float, c_vp, c_int],
    "ns2_linear_bf16_add_rmsnorm": [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_float],
}
_RESTYPES = {"ns2_last_error": ctypes.c_char_p, "ns2_get_stream": c_vp, "ns2_pool_round": c_size,
             "ns2_attention_vpack_bytes": c_size}


class NS2Error(RuntimeError):
    pass


def _ptr(x):
    """Device address of a tensor-like (``data_ptr()``), an int, or None -> NULL."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


class Lib:
    """Loaded libns2.so with checked calls."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise NS2Error(f"{path} is not built: run `make -C nanosaur2-web_amd`")
        self.path = path
        self.dll = ctypes.CDLL(path)
        for name, args in SIGNATURES.items():
            fn = getattr(self.dll, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, c_int)

    def exported(self):
        return [n for n in SIGNATURES if hasattr(self.dll, n)]

    def error(self) -> str:
        return self.dll.ns2_last_error().decode()

    def call(self, name, *args):
        rc = getattr(self.dll, name)(*args)
        if rc != 0:
            raise NS2Error(f"{name} failed ({rc}): {self.error()}")
        return rc

    # ---- runtime
    def init(self, device: int = 0):
        self.call("ns2_init", device)

    def set_stream(self, stream_handle: int | None):
        self.call("ns2_set_stream", stream_handle)

    def sync(self):
        self.call("ns2_sync")

    def device_info(self):
        name = ctypes.create_string_buffer(256)
        cus, hbm = c_int(), c_size()
        self.call("ns2_device_info", name, 256, ctypes.byref(cus), ctypes.byref(hbm))
        return {"name": name.value.decode(), "compute_units": cus.value, "hbm_bytes": hbm.value}

    # recorded launch sequences (HIP graphs) on the library's stream
    def graph_begin(self):
        self.call("ns2_graph_begin")

    def graph_end(self) -> int:
        g = c_vp()
        self.call("ns2_graph_end", ctypes.byref(g))
        return g.value

    def graph_launch(self, g):
        self.call("ns2_graph_launch", g)

    def graph_destroy(self, g):
        self.call("ns2_graph_destroy", g)

    def event(self):
        ev = c_vp()
        self.call("ns2_event_create", ctypes.byref(ev))
        return ev.value

    def record(self, ev):
        self.call("ns2_event_record", ev)

    def elapsed_ms(self, a, b) -> float:
        ms = c_float()
        self.call("ns2_event_elapsed", a, b, ctypes.byref(ms))
        return ms.value

    def profile(self, on: bool):
        self.call("ns2_profile_enable", int(on))

    def profile_reset(self):
        self.call("ns2_profile_reset")

    def profile_report(self) -> dict:
        """{kernel: {"count": n, "ms": total}} since the last reset."""
        import json

        buf = ctypes.create_string_buffer(1 << 16)
        self.call("ns2_profile_report", buf, 1 << 16)
        return json.loads(buf.value.decode())

    # ---- ops (argument meaning as in include/ns2.h)
    def hadamard256(self, x, y, groups):
        self.call("ns2_hadamard256", _ptr(x), _ptr(y), groups)

    def rotate_f16(self, x, ldx, y, ldy, rows, cols, tiled=False):
        self.call("ns2_rotate_f16", _ptr(x), ldx, _ptr(y), ldy, rows, cols, int(tiled))

    def tile_i8_weight(self, W, Wt, N, K):
        self.call("ns2_tile_i8_weight", _ptr(W), _ptr(Wt), N, K)

    def tile_i8_weight_glu(self, W, Wt, N, K):
        self.call("ns2_tile_i8_weight_glu", _ptr(W), _ptr(Wt), N, K)

    # lora = (lora_a fp16 [R, K], lora_b fp16 [N, R], R) selects the *_lora entry point
    def linear_i8_glu_rot_tiled(self, At, Wt, scale, Y, M, N, K, *, bias=None, alpha=1.0, act="silu", lora=None):
        args = [_ptr(At), _ptr(Wt), _ptr(scale), _ptr(bias), _ptr(Y), M, N, K, alpha, ACT[act]]
        self._linear("ns2_linear_i8_glu_rot_tiled", args, lora)

    def linear_i8_tiled(self, At, Wt, scale, C, M, N, K, *, bias=None, ldc=None, cOff=0, alpha=1.0,
                        act="none", resid=False, gate=None, gOff=0, lora=None):
        args = [_ptr(At), _ptr(Wt), _ptr(scale), _ptr(bias), _ptr(C), M, N, K,
                N if ldc is None else ldc, cOff, alpha, ACT[act], int(resid), _ptr(gate), gOff]
        self._linear("ns2_linear_i8_tiled", args, lora)

    def tile_bf16_weight(self, W, Wt, N, K):
        self.call("ns2_tile_bf16_weight", _ptr(W), _ptr(Wt), N, K)

    def linear_f16w_tiled(self, At, Wt, C, M, N, K, *, bias=None, ldc=None, cOff=0, alpha=1.0, act="none",
                          resid=False, gate=None, gOff=0, lora=None):
        args = [_ptr(At), _ptr(Wt), _ptr(bias), _ptr(C), M, N, K, N if ldc is None else ldc, cOff, alpha, ACT[act],
                int(resid), _ptr(gate), gOff]
        self._linear("ns2_linear_f16w_tiled", args, lora)

    def to_tiled_f16(self, x, ldx, y, rows, cols, *, sub=None, ldsub=0):
        self.call("ns2_to_tiled_f16", _ptr(x), ldx, _ptr(sub), ldsub, _ptr(y), rows, cols)

    def norm_mod_f16(self, x, mod, shiftOff, scaleOff, rows, cols, weight, y, eps=1e-6, tiled=True):
        self.call("ns2_norm_mod_f16", _ptr(x), _ptr(mod), shiftOff, scaleOff, rows, cols, _ptr(weight), eps, _ptr(y),
                  int(tiled))

    def linear_i8_tiled_vpack(self, At, Wt, scale, C, M, N, K, vpk, *, vcol0, H, D, Lk, bias=None, ldc=None,
                              cOff=0, alpha=1.0, act="none", lora=None):
        """ns2_linear_i8_tiled_vpack: columns [vcol0, N) go to vpk as the attention's packed values
        of keys [0, M)."""
        a, b, r = lora if lora is not None else (None, None, 0)
        self.call("ns2_linear_i8_tiled_vpack", _ptr(At), _ptr(Wt), _ptr(scale), _ptr(bias), _ptr(C), M, N, K,
                  N if ldc is None else ldc, cOff, alpha, ACT[act], _ptr(a), _ptr(b), r, _ptr(vpk), vcol0, H, D, Lk)

    def attention_vpack_bytes(self, Lk, H, D):
        return int(self.dll.ns2_attention_vpack_bytes(Lk, H, D))

    def linear_i8(self, A, a_fmt, lda, W, scale, C, M, N, K, *, bias=None, add=None, ldc=None,
                  cOff=0, alpha=1.0, act="none", resid=False, gate=None, gOff=0, lora=None):
        args = [_ptr(A), a_fmt, lda, _ptr(W), _ptr(scale), _ptr(bias), _ptr(add),
                _ptr(C), M, N, K, N if ldc is None else ldc, cOff, alpha, ACT[act], int(resid),
                _ptr(gate), gOff]
        self._linear("ns2_linear_i8", args, lora)

    def linear_bf16(self, A, lda, W, C, M, N, K, *, bias=None, add=None, ldc=None, cOff=0,
                    alpha=1.0, act="none", resid=False, gate=None, gOff=0, lora=None):
        args = [_ptr(A), lda, _ptr(W), _ptr(bias), _ptr(add), _ptr(C), M, N, K,
                N if ldc is None else ldc, cOff, alpha, ACT[act], int(resid), _ptr(gate), gOff]
        self._linear("ns2_linear_bf16", args, lora)

    def _linear(self, name, args, lora):
        if lora is None:
            self.call(name, *args)
        else:
            a, b, r = lora
            self.call(name + "_lora", *args, _ptr(a), _ptr(b), r)

    def attention(self, q, k, v, o, *, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff=0, kOff=0, vOff=0,
                  oOff=0, batch=1, qBatch=0, kBatch=0, vBatch=0, oBatch=0, scale=None,
                  key_bias=None, biasStart=0, biasBatch=0, q_norm=None, k_norm=None, eps=1e-6,
                  rope_cs=None, sin_off=0, rope_rows=0, noalloc=False):
        """ns2_attention, or with noalloc=True ns2_attention_noalloc (same arguments; its
        scratch is the library's fixed device array, no allocation)."""
        if scale is None:
            scale = 1.0 / D ** 0.5
        fn = "ns2_attention_noalloc" if noalloc else "ns2_attention"
        self.call(fn, _ptr(q), _ptr(k), _ptr(v), _ptr(o), batch, Lq, Lk, H, D, ldq, ldk,
                  ldv, ldo, qOff, kOff, vOff, oOff, qBatch, kBatch, vBatch, oBatch, scale,
                  _ptr(key_bias), biasStart, biasBatch, _ptr(q_norm), _ptr(k_norm), eps,
                  _ptr(rope_cs), sin_off, rope_rows)

    def attention_text(self, q, k, v, o, *, Lq, Lk, H, D, ldq, ldk, ldv, ldo, k_text, v_text, ld_text, text_start,
                       qOff=0, kOff=0, vOff=0, oOff=0, scale=None, key_bias=None, biasStart=0, q_norm=None,
                       k_norm=None, eps=1e-6, rope_cs=None, sin_off=0, rope_rows=0):
        """ns2_attention_text: key/value rows from text_start on come from k_text / v_text (row
        stride ld_text)."""
        if scale is None:
            scale = 1.0 / D ** 0.5
        self.call("ns2_attention_text", _ptr(q), _ptr(k), _ptr(v), _ptr(o), Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff,
                  kOff, vOff, oOff, scale, _ptr(key_bias), biasStart, _ptr(q_norm), _ptr(k_norm), eps, _ptr(rope_cs),
                  sin_off, rope_rows, _ptr(k_text), _ptr(v_text), ld_text, text_start)

    def attention_vpacked(self, q, k, v, o, vpk, v_rows, *, Lq, Lk, H, D, ldq, ldk, ldv, ldo, k_text=None,
                          v_text=None, ld_text=0, text_start=0, qOff=0, kOff=0, vOff=0, oOff=0, scale=None,
                          key_bias=None, biasStart=0, q_norm=None, k_norm=None, eps=1e-6, rope_cs=None, sin_off=0,
                          rope_rows=0):
        """ns2_attention_vpacked: the values of keys [0, v_rows) are already packed in vpk."""
        if scale is None:
            scale = 1.0 / D ** 0.5
        self.call("ns2_attention_vpacked", _ptr(q), _ptr(k), _ptr(v), _ptr(o), Lq, Lk, H, D, ldq, ldk, ldv, ldo,
                  qOff, kOff, vOff, oOff, scale, _ptr(key_bias), biasStart, _ptr(q_norm), _ptr(k_norm), eps,
                  _ptr(rope_cs), sin_off, rope_rows, _ptr(k_text), _ptr(v_text), ld_text, text_start, _ptr(vpk),
                  v_rows)

    def attention_rows(self, q, k, v, o, *, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff=0, kOff=0, vOff=0,
                       group=1, causal=False):
        self.call("ns2_attention_rows", _ptr(q), _ptr(k), _ptr(v), _ptr(o), Lq, Lk, H, D, ldq, ldk, ldv,
                  ldo, qOff, kOff, vOff, group, int(causal))

    def attention_rows_f16kv_oproj(self, q, k, v, wo_tiled, part, *, Lq, Lk, H, D, ldq, ldk, ldv, N, qOff=0,
                                   kOff=0, vOff=0, group=1, causal=False):
        """attention_rows_f16kv with each head's share of the output projection into part [H, Lq, N]."""
        self.call("ns2_attention_rows_f16kv_oproj", _ptr(q), _ptr(k), _ptr(v), _ptr(wo_tiled), _ptr(part), Lq, Lk,
                  H, D, ldq, ldk, ldv, qOff, kOff, vOff, group, int(causal), N)

    def parts_add_rmsnorm_tiled(self, part, splits, bias, x, w_add, w_out, yt, M, N, eps=1e-6):
        self.call("ns2_parts_add_rmsnorm_tiled", _ptr(part), splits, _ptr(bias), _ptr(x), _ptr(w_add), _ptr(w_out),
                  _ptr(yt), M, N, eps)

    def linear_f16w_tiled_head_norm_f16kv(self, At, Wt, bias, C, M, N, K, w1, H1, w2, H2, D, kv16, ldkv, cs=None,
                                          sin_off=0, rope_rows=0, eps=1e-6):
        self.call("ns2_linear_f16w_tiled_head_norm_f16kv", _ptr(At), _ptr(Wt), _ptr(bias), _ptr(C), M, N, K,
                  _ptr(w1), H1, _ptr(w2), H2, D, _ptr(cs), sin_off, rope_rows, eps, _ptr(kv16), ldkv)

    def linear_f16w_tiled_glu_down(self, At, Wt, bias, M, N, K, wd_tiled, Nd, part, act="gelu_tanh"):
        self.call("ns2_linear_f16w_tiled_glu_down", _ptr(At), _ptr(Wt), _ptr(bias), M, N, K, ACT[act],
                  _ptr(wd_tiled), Nd, _ptr(part))

    def parts_add_rmsnorm(self, part, splits, bias, x, w_add, w_out, y, M, N, eps=1e-6):
        self.call("ns2_parts_add_rmsnorm", _ptr(part), splits, _ptr(bias), _ptr(x), _ptr(w_add), _ptr(w_out),
                  _ptr(y), M, N, eps)

    def attention_rows_f16kv(self, q, k, v, o, *, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff=0, kOff=0, vOff=0,
                             group=1, causal=False):
        """attention_rows with fp16 k and v (their strides and offsets in fp16 elements)."""
        self.call("ns2_attention_rows_f16kv", _ptr(q), _ptr(k), _ptr(v), _ptr(o), Lq, Lk, H, D, ldq, ldk, ldv,
                  ldo, qOff, kOff, vOff, group, int(causal))

    def head_norm(self, X, w, L, H, D, ld, colOff=0, rowOff=0, cs=None, sinOff=0, eps=1e-6):
        self.call("ns2_head_norm", _ptr(X), _ptr(w), L, H, D, ld, colOff, rowOff, _ptr(cs), sinOff, eps)

    def head_norm2(self, X, w1, H1, w2, H2, L, D, ld, colOff=0, rowOff=0, cs=None, sinOff=0, eps=1e-6):
        self.call("ns2_head_norm2", _ptr(X), _ptr(w1), H1, _ptr(w2), H2, L, D, ld, colOff, rowOff, _ptr(cs),
                  sinOff, eps)

    def norm_mod(self, x, mod, shiftOff, scaleOff, rows, cols, weight, y, eps=1e-6):
        self.call("ns2_norm_mod", _ptr(x), _ptr(mod), shiftOff, scaleOff, rows, cols, _ptr(weight), eps, _ptr(y))

    def norm_mod_rotate_f16(self, x, mod, shiftOff, scaleOff, rows, cols, weight, y, eps=1e-6, tiled=False):
        self.call("ns2_norm_mod_rotate_f16", _ptr(x), _ptr(mod), shiftOff, scaleOff, rows, cols,
                  _ptr(weight), eps, _ptr(y), int(tiled))

    def glu(self, x, y, rows, I, act="silu"):
        self.call("ns2_glu", _ptr(x), _ptr(y), rows, I, ACT[act])

    def glu_rotate_f16(self, x, y, rows, I, act="silu", tiled=False):
        self.call("ns2_glu_rotate_f16", _ptr(x), _ptr(y), rows, I, ACT[act], int(tiled))

    def elementwise(self, op, a, b, y, n):
        self.call("ns2_elementwise", EW[op], _ptr(a), _ptr(b), _ptr(y), n)

    def accumulate(self, y, a, n):
        self.call("ns2_accumulate", _ptr(y), _ptr(a), n)

    def add_rows(self, a, b, y, rows, n):
        self.call("ns2_add_rows", _ptr(a), _ptr(b), _ptr(y), rows, n)

    def row_sum(self, x, w, y, rows, N, scale=1.0):
        self.call("ns2_row_sum", _ptr(x), _ptr(w), _ptr(y), rows, N, scale)

    def rmsnorm(self, x, w, y, rows, cols, eps=1e-6):
        self.call("ns2_rmsnorm", _ptr(x), _ptr(w), _ptr(y), rows, cols, eps)

    def transpose(self, x, y, rows, cols):
        self.call("ns2_transpose", _ptr(x), _ptr(y), rows, cols)

    def add_rmsnorm(self, x, a, w_add, w_out, y, rows, cols, eps=1e-6):
        self.call("ns2_add_rmsnorm", _ptr(x), _ptr(a), _ptr(w_add), _ptr(w_out), _ptr(y), rows, cols, eps)

    def linear_bf16_head_norm(self, A, lda, W, bias, C, M, N, K, w1, H1, w2, H2, D, cs=None, sin_off=0,
                              rope_rows=0, eps=1e-6):
        self.call("ns2_linear_bf16_head_norm", _ptr(A), lda, _ptr(W), _ptr(bias), _ptr(C), M, N, K, _ptr(w1), H1,
                  _ptr(w2), H2, D, _ptr(cs), sin_off, rope_rows, eps)

    def linear_bf16_head_norm_f16kv(self, A, lda, W, bias, C, M, N, K, w1, H1, w2, H2, D, kv16, ldkv, cs=None,
                                    sin_off=0, rope_rows=0, eps=1e-6):
        """linear_bf16_head_norm with heads H1.. stored as fp16 in kv16 [M, ldkv] (a device address,
        or a tensor)."""
        self.call("ns2_linear_bf16_head_norm_f16kv", _ptr(A), lda, _ptr(W), _ptr(bias), _ptr(C), M, N, K,
                  _ptr(w1), H1, _ptr(w2), H2, D, _ptr(cs), sin_off, rope_rows, eps, _ptr(kv16), ldkv)

    def linear_bf16_glu(self, A, lda, W, bias, Y, M, N, K, act="gelu_tanh"):
        self.call("ns2_linear_bf16_glu", _ptr(A), lda, _ptr(W), _ptr(bias), _ptr(Y), M, N, K, ACT[act])

    def linear_bf16_glu_down(self, A, lda, W, bias, M, N, K, wd_tiled, Nd, part, act="gelu_tanh"):
        """linear_bf16_glu and the next linear's shares per 128-column group into part [N/256, M, Nd]."""
        self.call("ns2_linear_bf16_glu_down", _ptr(A), lda, _ptr(W), _ptr(bias), M, N, K, ACT[act], _ptr(wd_tiled), Nd,
                  _ptr(part))

    def linear_bf16_add_rmsnorm(self, A, lda, W, bias, x, w_add, w_out, y, M, N, K, eps=1e-6):
        self.call("ns2_linear_bf16_add_rmsnorm", _ptr(A), lda, _ptr(W), _ptr(bias), _ptr(x), _ptr(w_add),
                  _ptr(w_out), _ptr(y), M, N, K, eps)


_LIB = None


def load(device: int = 0, stream_handle: int | None = None) -> Lib:
    """The process-wide library handle, initialised on `device`."""
    global _LIB
    if _LIB is None:
        lib = Lib()
        lib.init(device)
        _LIB = lib
    if stream_handle is not None:
        _LIB.set_stream(stream_handle)
    return _LIB
