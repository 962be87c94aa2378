"""TEST INFRASTRUCTURE, NOT PRODUCT: the CPU restatement of tgo's batched path.

`oracle.lib` is liboracle.so (oracle.c, built by oracle/Makefile) loaded with
ctypes; `oracle.host` is the pure-Python restatement of the host integer
logic. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
import this package, and only as the checker or the timed CPU baseline.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

FORM_F16, FORM_I8, FORM_I4_TGO, FORM_I4_SYM = 0, 1, 2, 3


def build():
    """Compile oracle.c (gcc, OpenMP) into oracle/liboracle.so."""
    subprocess.check_call(["make", "-s", "-B", "-C", HERE])


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    P, I, U64, D, F = (ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_double,
                       ctypes.c_float)
    sig = {
        "orc_splitmix64": (U64, [U64]),
        "orc_hash3": (U64, [U64, U64, U64]),
        "orc_normal": (D, [U64, U64, U64]),
        "orc_synth_normal_f32": (None, [U64, U64, ctypes.c_size_t, D, P]),
        "orc_synth_normal_f16": (None, [U64, U64, ctypes.c_size_t, D, P]),
        "orc_f32_to_f16_bits": (ctypes.c_uint16, [F, P]),
        "orc_f32_to_f16_ieee": (ctypes.c_uint16, [F]),
        "orc_f16_to_f32": (F, [ctypes.c_uint16]),
        "orc_to_f16": (ctypes.c_size_t, [P, P, ctypes.c_size_t]),
        "orc_transpose": (None, [P, P, I, I]),
        "orc_f16_ieee_bits_array": (None, [P, P, ctypes.c_size_t]),
        "orc_f16_loader_bits_array": (None, [P, P, ctypes.c_size_t]),
        "orc_permute_heads": (I, [P, ctypes.c_size_t, I, I]),
        "orc_quantize_int8": (None, [P, ctypes.c_size_t, P, P]),
        "orc_dequant_int8": (None, [P, P, ctypes.c_size_t, P]),
        "orc_quantize_int4_tgo": (None, [P, ctypes.c_size_t, P, P, P]),
        "orc_dequant_int4_tgo": (None, [P, P, P, ctypes.c_size_t, P]),
        "orc_dequant_int4_sym": (None, [P, P, I, I, P]),
        "orc_synth_int4_sym": (None, [U64, U64, I, I, D, P, P]),
        "orc_int4_tgo_bound": (D, [P, P, P, I, I, I]),
        "orc_rmsnorm_f64": (None, [P, P, I, I, D, P]),
        "orc_matmul_f64": (None, [P, P, I, I, I, P]),
        "orc_silu_f64": (None, [P, I, P]),
        "orc_swiglu_f64": (None, [P, P, I, P]),
        "orc_softmax_f64": (None, [P, I, P]),
        "orc_gather_rows_f64": (None, [P, I, I, P, I, P]),
        "orc_rope_f64": (None, [P, I, I, I, D, P, I, P]),
        "orc_attention_f64": (None, [P, P, P, I, I, I, I, I, D, I, P]),
        "orc_ragged_attention_f64": (None, [P, I, I, I, I, P, P, P, P, I, P, P, P, I, I, D, P, P]),
        "orc_model_new": (P, [I, I, I, I, I, I, I, F, F, I, I]),
        "orc_model_free": (None, [P]),
        "orc_model_weight": (I, [P, ctypes.c_char_p, I, I, I, P, P, P]),
        "orc_model_gain": (I, [P, ctypes.c_char_p, P, I]),
        "orc_model_synth": (I, [P, U64, I, D, I]),
        "orc_model_kv": (None, [P, P, P]),
        "orc_synth_gain": (None, [U64, U64, ctypes.c_size_t, P]),
        "orc_model_set_fault": (I, [P, I]),
        "orc_model_step": (I, [P, I, I, P, P, P, P, P, P, P, P, I, P, I]),
        "orc_cpu_ragged_attention": (None, [P, I, I, I, I, P, P, I, P, P, P, I, I, F, P]),
        "orc_cpu_linear": (I, [P, I, I, I, I, P, P, P, P]),
        "orc_num_threads": (I, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def ptr(a):
    """ctypes pointer of a numpy array (None passes NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def f16_bits(x):
    """Loader rule narrowing (weights/convert.go:153-180) of an array -> uint16."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib.orc_to_f16(ptr(x), ptr(out), x.size)
    return out


def f16_to_f32(bits):
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def synth_normal_f32(seed, stream, n, sigma):
    out = np.empty(n, dtype=np.float32)
    lib.orc_synth_normal_f32(seed, stream, n, sigma, ptr(out))
    return out


def synth_normal_f16(seed, stream, n, sigma):
    out = np.empty(n, dtype=np.uint16)
    lib.orc_synth_normal_f16(seed, stream, n, sigma, ptr(out))
    return out


def synth_gain(seed, stream, n):
    """The synthesizer's gains: multiples of 1/8 in [-2, 2)."""
    out = np.empty(n, dtype=np.float32)
    lib.orc_synth_gain(seed, stream, n, ptr(out))
    return out


# planted mistakes (orc_model_set_fault), for the sensitivity tests
FAULT_NONE, FAULT_QKNORM_AFTER_ROPE, FAULT_QK_UNIT_GAIN, FAULT_K_TAKES_Q_GAIN = 0, 1, 2, 3
FAULT_QK_GAIN_AFTER_ROPE, FAULT_NORM_UNIT_GAIN, FAULT_FINAL_UNIT_GAIN = 4, 5, 6


def synth_int4_sym(seed, stream, K, N, sigma):
    qw = np.empty((K // 8, N), dtype=np.uint32)
    sc = np.empty((K // 32, N), dtype=np.uint16)
    lib.orc_synth_int4_sym(seed, stream, K, N, sigma, ptr(qw), ptr(sc))
    return qw, sc


def dequant(form, K, N, plane, scales=None, zeros=None):
    """Dequantize a [K,N] weight in any form to float32 [K,N]."""
    out = np.empty((K, N), dtype=np.float32)
    n = K * N
    if form == FORM_F16:
        return f16_to_f32(plane).reshape(K, N)
    if form == FORM_I8:
        lib.orc_dequant_int8(ptr(plane), ptr(scales), n, ptr(out))
    elif form == FORM_I4_TGO:
        lib.orc_dequant_int4_tgo(ptr(plane), ptr(scales), ptr(zeros), n, ptr(out))
    else:
        lib.orc_dequant_int4_sym(ptr(plane), ptr(scales), K, N, ptr(out))
    return out


def cpu_linear(x, form, K, N, plane, scales=None, zeros=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    lib.orc_cpu_linear(ptr(x), M, K, N, form, ptr(plane), ptr(scales), ptr(zeros), ptr(y))
    return y


def ragged_attention_f64(q, H, Hkv, dh, k, v, lengths, extents, pages, max_pages, block, scale,
                         f16_cache=True):
    """raggedOracle (ragged_test.go:151-208); returns (out [T,H,dh] f64, budget dict)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    T = q.shape[0]
    out = np.zeros((T, H, dh), dtype=np.float64)
    b3 = np.zeros(3, dtype=np.float64)
    u = lambda a: np.ascontiguousarray(a, dtype=np.uint32)
    lengths, extents, pages = u(lengths), u(extents), u(pages)
    if f16_cache:
        k16 = np.ascontiguousarray(k, dtype=np.uint16)
        v16 = np.ascontiguousarray(v, dtype=np.uint16)
        lib.orc_ragged_attention_f64(ptr(q), T, H, Hkv, dh, ptr(k16), ptr(v16), None, None,
                                     len(lengths), ptr(lengths), ptr(extents), ptr(pages),
                                     max_pages, block, scale, ptr(out), ptr(b3))
    else:
        k32 = np.ascontiguousarray(k, dtype=np.float32)
        v32 = np.ascontiguousarray(v, dtype=np.float32)
        lib.orc_ragged_attention_f64(ptr(q), T, H, Hkv, dh, None, None, ptr(k32), ptr(v32),
                                     len(lengths), ptr(lengths), ptr(extents), ptr(pages),
                                     max_pages, block, scale, ptr(out), ptr(b3))
    return out, dict(value=b3[0], score=b3[1], positions=int(b3[2]))


def cpu_ragged_attention(q, H, Hkv, dh, k16, v16, lengths, extents, pages, max_pages, block,
                         scale):
    q = np.ascontiguousarray(q, dtype=np.float32)
    T = q.shape[0]
    out = np.zeros((T, H, dh), dtype=np.float32)
    u = lambda a: np.ascontiguousarray(a, dtype=np.uint32)
    lengths, extents, pages = u(lengths), u(extents), u(pages)
    lib.orc_cpu_ragged_attention(ptr(q), T, H, Hkv, dh, ptr(np.ascontiguousarray(k16)),
                                 ptr(np.ascontiguousarray(v16)), len(lengths), ptr(lengths),
                                 ptr(extents), ptr(pages), max_pages, block, scale, ptr(out))
    return out


class CPUModel:
    """The f32 CPU path over a whole Qwen3-shaped model (orc_model_*)."""

    def __init__(self, layers, hidden, heads, kv_heads, head_dim, ffn, vocab, eps, theta,
                 block, capacity):
        self.cfg = dict(layers=layers, hidden=hidden, heads=heads, kv_heads=kv_heads,
                        head_dim=head_dim, ffn=ffn, vocab=vocab, eps=eps, theta=theta,
                        block=block, capacity=capacity)
        self.h = lib.orc_model_new(layers, hidden, heads, kv_heads, head_dim, ffn, vocab, eps,
                                   theta, block, capacity)

    def close(self):
        if self.h:
            lib.orc_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def synth(self, seed, form, sigma, layers_limit=-1):
        lib.orc_model_synth(self.h, seed, form, sigma, layers_limit)

    def weight(self, port, form, K, N, plane, scales=None, zeros=None):
        rc = lib.orc_model_weight(self.h, port.encode(), form, K, N, ptr(plane), ptr(scales),
                                  ptr(zeros))
        assert rc == 0, port

    def gain(self, port, g):
        g = np.ascontiguousarray(g, dtype=np.float32)
        assert lib.orc_model_gain(self.h, port.encode(), ptr(g), g.size) == 0

    def set_fault(self, fault):
        assert lib.orc_model_set_fault(self.h, fault) == 0

    def kv(self):
        kp, vp = ctypes.c_void_p(), ctypes.c_void_p()
        lib.orc_model_kv(self.h, ctypes.byref(kp), ctypes.byref(vp))
        c = self.cfg
        n = c["layers"] * c["capacity"] * c["kv_heads"] * c["head_dim"]
        k = np.ctypeslib.as_array(ctypes.cast(kp, ctypes.POINTER(ctypes.c_uint16)), shape=(n,))
        v = np.ctypeslib.as_array(ctypes.cast(vp, ctypes.POINTER(ctypes.c_uint16)), shape=(n,))
        return k, v

    def step(self, st, pages, max_pages, layers=-1):
        """st: dict of ports from host.new_batch_step; pages: flat [B*max_pages]."""
        u = lambda a: np.ascontiguousarray(a, dtype=np.uint32)
        ids, posq, posk, slots = u(st["ids"]), u(st["posq"]), u(st["posk"]), u(st["slots"])
        lengths, extents, last = u(st["lengths"]), u(st["extents"]), u(st["last"])
        pages = u(pages)
        B = len(lengths)
        logits = np.zeros((B, self.cfg["vocab"]), dtype=np.float32)
        lib.orc_model_step(self.h, len(ids), B, ptr(ids), ptr(posq), ptr(posk), ptr(slots),
                           ptr(lengths), ptr(extents), ptr(last), ptr(pages), max_pages,
                           ptr(logits), layers)
        return logits
