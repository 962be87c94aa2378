"""tgo_amd: the MI355X (gfx950) implementation of tgo's batched forward pass.

The product is libtgohip.so (tgo_amd/csrc, C ABI in include/tgohip.h). This
module loads it with ctypes and mirrors the reference's host-side API for the
path (model.NewBatchStep, nextStep/victim, prefix.Pool/Lease, Scheduler,
nn.Linear, tensor.Attention). Every call goes through the C ABI; a missing or
unbuilt library raises -- there is no CPU fallback.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtgohip.so")

FORM_F16, FORM_I8, FORM_I4_TGO, FORM_I4_SYM = 0, 1, 2, 3
F32, F16, F16X2 = 0, 1, 2
PROF_ATTN, PROF_QKV, PROF_O, PROF_GATEUP, PROF_DOWN, PROF_LMHEAD = range(6)
PROF_NAMES = ("attention", "qkv", "o", "gateup", "down", "lm_head")

EINVAL, ENOMEM, EDEVICE, ESTATE, EEXHAUSTED, ENOSLOT = -1, -2, -3, -4, -5, -6


class TgoError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


class ModelCfg(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_int32), ("hidden", ctypes.c_int32),
                ("heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32),
                ("head_dim", ctypes.c_int32), ("ffn", ctypes.c_int32),
                ("vocab", ctypes.c_int32), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("block", ctypes.c_int32)]


class BatchStepC(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_int32), ("batch", ctypes.c_int32),
                ("max_pages", ctypes.c_int32)] + [
        (n, ctypes.c_void_p) for n in ("ids", "posq", "posk", "slots", "lengths", "extents",
                                       "last", "pages")]


class Timings(ctypes.Structure):
    _fields_ = [("submit_ms", ctypes.c_double), ("device_ms", ctypes.c_double),
                ("readback_ms", ctypes.c_double)]


_lib = None


def lib():
    """The loaded libtgohip.so. Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("tgo_amd: %s is not built; run `python -m tgo_amd.build`" % LIB_PATH)
    L = ctypes.CDLL(LIB_PATH)
    P, I, U64, D, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_double, ctypes.c_float
    sig = {
        "tgohip_last_error": (ctypes.c_char_p, []),
        "tgohip_version": (ctypes.c_char_p, []),
        "tgohip_open": (P, [I]),
        "tgohip_close": (None, [P]),
        "tgohip_stream": (P, [P]),
        "tgohip_sync": (I, [P]),
        "tgohip_set_stream": (I, [P, P]),
        "tgohip_set_precision": (I, [P, I]),
        "tgohip_set_cascade": (I, [P, I]),
        "tgohip_use_own_stream": (I, [P]),
        "tgohip_config": (I, [P, ctypes.POINTER(ModelCfg)]),
        "tgohip_weight": (I, [P, ctypes.c_char_p, I, I, I, P, P, P]),
        "tgohip_weight_f32": (I, [P, ctypes.c_char_p, I, I, I, P]),
        "tgohip_weight_upload_f32": (I, [P, I, I, I, P, P]),
        "tgohip_gain": (I, [P, ctypes.c_char_p, P, I]),
        "tgohip_synth_weights": (I, [P, U64, I, D]),
        "tgohip_kv_alloc": (I, [P, I]),
        "tgohip_kv_pointers": (I, [P, P, P, P]),
        "tgohip_step": (I, [P, ctypes.POINTER(BatchStepC), P, P, ctypes.POINTER(Timings)]),
        "tgohip_paged_attention": (I, [P, P, I, I, I, I, I, P, P, I, I, P, P, P, I, I, F, P, I]),
        "tgohip_paged_attention_replay": (I, [P, P, I, I, I, I, P, P, I, I, P, P, P, I, I, F, P, I, I]),
        "tgohip_weight_upload": (I, [P, I, I, I, P, P, P, P]),
        "tgohip_weight_synth": (I, [P, I, I, I, U64, U64, D, P]),
        "tgohip_weight_free": (I, [P, I]),
        "tgohip_linear": (I, [P, I, P, I, I, P, I]),
        "tgohip_linear_noalloc": (I, [P, I, P, I, I, P, I]),
        "tgohip_linear_workspace": (I, [P, I, I, I, P]),
        "tgohip_dequant": (I, [P, I, P]),
        "tgohip_dequant_f16": (I, [P, I, P]),
        "tgohip_greedy": (I, [P, P, I, I, P, P]),
        "tgohip_step_margins": (I, [P, P, I]),
        "tgohip_new_batch_step": (I, [I, I, I, I, I, P, P, P, P, P, I, I, I, P, P, P, P, P, P, P]),
        "tgohip_next_step": (I, [I, P, P, P, I, I, P, P, P, P, P, P]),
        "tgohip_victim": (I, [I, P, P, P, P]),
        "tgohip_sha256": (I, [P, ctypes.c_size_t, P]),
        "tgohip_pool_new": (P, [I, I, I]),
        "tgohip_pool_free": (None, [P]),
        "tgohip_pool_stats": (None, [P, P]),
        "tgohip_pool_acquire": (I, [P, P, I, ctypes.c_char_p, ctypes.c_char_p, I, P]),
        "tgohip_lease_blocks": (I, [P, P, I]),
        "tgohip_lease_reused": (I, [P]),
        "tgohip_lease_len": (I, [P]),
        "tgohip_lease_grow": (I, [P, I]),
        "tgohip_lease_commit": (I, [P, P, I]),
        "tgohip_lease_publish": (I, [P, I]),
        "tgohip_lease_release": (None, [P]),
        "tgohip_lease_free": (None, [P]),
        "tgohip_sched_new": (P, [P, I, I, I, I]),
        "tgohip_sched_free": (None, [P]),
        "tgohip_sched_admit": (I, [P, P, I, I]),
        "tgohip_sched_finish": (I, [P, I]),
        "tgohip_sched_evict": (I, [P]),
        "tgohip_sched_feed": (I, [P, I, I]),
        "tgohip_sched_length": (I, [P, I]),
        "tgohip_sched_step": (I, [P, P, P, P, P, P, ctypes.POINTER(Timings)]),
        "tgohip_sched_admit_prefilled": (I, [P, P, I, I, I]),
        "tgohip_sched_prefilling": (I, [P]),
        "tgohip_sched_live": (I, [P]),
        "tgohip_sched_last_step": (I, [P, P, P, P, P, P, P, P, P, P, P, P]),
        "tgohip_sched_set_overlap": (I, [P, I]),
        "tgohip_sched_submit": (I, [P, P, P, P, P]),
        "tgohip_sched_collect": (I, [P, P, P, P, ctypes.POINTER(Timings)]),
        "tgohip_set_profile": (I, [P, I]),
        "tgohip_profile_read": (I, [P, P, P, P]),
        "tgohip_set_profile_kernels": (I, [P, I, I]),
        "tgohip_profile_read_kernel": (I, [P, I, P, P, P, P]),
        "tgohip_kv_synth": (I, [P, U64, D, I]),
        "tgohip_probe_peaks": (I, [P, ctypes.c_size_t, I, P, P]),
        "tgohip_to_f16": (ctypes.c_size_t, [P, P, ctypes.c_size_t]),
        "tgohip_quantize_int8": (None, [P, ctypes.c_size_t, P, P]),
        "tgohip_quantize_int4": (None, [P, ctypes.c_size_t, P, P, P]),
        "tgohip_get_config": (I, [P, ctypes.POINTER(ModelCfg)]),
        "tgohip_st_open": (P, [ctypes.c_char_p]),
        "tgohip_st_close": (None, [P]),
        "tgohip_st_count": (I, [P]),
        "tgohip_st_entry": (I, [P, I, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p),
                                ctypes.POINTER(ctypes.c_int), P, ctypes.POINTER(ctypes.c_int64),
                                ctypes.POINTER(ctypes.c_int64)]),
        "tgohip_st_read": (ctypes.c_int64, [P, ctypes.c_char_p, P, ctypes.c_int64]),
        "tgohip_st_set_max_header": (None, [ctypes.c_int64]),
        "tgohip_repo_open": (P, [ctypes.c_char_p]),
        "tgohip_repo_close": (None, [P]),
        "tgohip_repo_has": (I, [P, ctypes.c_char_p]),
        "tgohip_repo_plane": (I, [P, ctypes.c_char_p, I, I, P, ctypes.c_int64]),
        "tgohip_load_qwen3": (I, [P, P, I, I, ctypes.POINTER(ctypes.c_int64)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error():
    return lib().tgohip_last_error().decode()


def check(rc):
    if rc < 0:
        raise TgoError(rc, last_error())
    return rc


def ptr(a):
    """A ctypes pointer for a numpy array, a torch tensor, an int address or None."""
    if a is None:
        return None
    if isinstance(a, int):
        return ctypes.c_void_p(a)
    if isinstance(a, np.ndarray):
        assert a.flags["C_CONTIGUOUS"], "arrays passed to the C ABI are contiguous"
        return a.ctypes.data_as(ctypes.c_void_p)
    # torch tensor
    assert a.is_contiguous(), "tensors passed to the C ABI are contiguous"
    return ctypes.c_void_p(a.data_ptr())


def u32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def i32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


# ---------------------------------------------------------------------------
# host mirrors
# ---------------------------------------------------------------------------

def new_batch_step(vocab, heads, kv_heads, rows, members, block, capacity):
    """model.NewBatchStep (model/batch.go:66-152). members: [(tokens, first, pages)]."""
    B = len(members)
    tokens = i32([t for m in members for t in m[0]] or [0])
    counts = i32([len(m[0]) for m in members])
    first = i32([m[1] for m in members])
    maxp = max([len(m[2]) for m in members] + [1])
    pages = np.zeros((B, maxp), dtype=np.int32)
    for i, m in enumerate(members):
        pages[i, :len(m[2])] = m[2]
    plen = i32([len(m[2]) for m in members])
    rows_ = max(rows, 0)
    out = dict(ids=np.zeros(rows_, np.uint32), posq=np.zeros(rows_ * heads, np.uint32),
               posk=np.zeros(rows_ * kv_heads, np.uint32), slots=np.zeros(rows_, np.uint32),
               lengths=np.zeros(B, np.uint32), extents=np.zeros(B, np.uint32),
               last=np.zeros(B, np.uint32))
    check(lib().tgohip_new_batch_step(vocab, heads, kv_heads, rows, B, ptr(tokens), ptr(counts),
                                      ptr(first), ptr(pages), ptr(plen), maxp, block, capacity,
                                      ptr(out["ids"]), ptr(out["posq"]), ptr(out["posk"]),
                                      ptr(out["slots"]), ptr(out["lengths"]), ptr(out["extents"]),
                                      ptr(out["last"])))
    return out


def next_step(live, prompt_len, prefilled, chunk, rows):
    """nextStep (schedule.go:80-118) -> ([(slot, start|-1, count)], prefill, decode)."""
    n = len(live)
    ws, wst, wc = (np.zeros(max(n, 1), np.int32) for _ in range(3))
    nw, pf, dc = (ctypes.c_int32() for _ in range(3))
    check(lib().tgohip_next_step(n, ptr(i32(live or [0])), ptr(i32(prompt_len or [0])),
                                 ptr(i32(prefilled or [0])), chunk, rows, ptr(ws), ptr(wst), ptr(wc),
                                 ctypes.byref(nw), ctypes.byref(pf), ctypes.byref(dc)))
    work = [(int(ws[i]), int(wst[i]), int(wc[i])) for i in range(nw.value)]
    return work, pf.value, dc.value


def victim(live, prompt_len, prefilled, arrived):
    n = len(live)
    return lib().tgohip_victim(n, ptr(i32(live or [0])), ptr(i32(prompt_len or [0])),
                               ptr(i32(prefilled or [0])),
                               ptr(np.ascontiguousarray(np.asarray(arrived or [0], np.uint64))))


def sha256(data: bytes):
    buf = np.frombuffer(data, dtype=np.uint8).copy() if data else np.zeros(1, np.uint8)
    out = np.zeros(32, np.uint8)
    lib().tgohip_sha256(ptr(buf), len(data), ptr(out))
    return out.tobytes()


class Lease:
    """prefix.Lease over the C ABI."""

    def __init__(self, h):
        self.h = h

    def blocks(self):
        n = lib().tgohip_lease_blocks(self.h, None, 0)
        out = np.zeros(max(n, 1), np.int32)
        lib().tgohip_lease_blocks(self.h, ptr(out), n)
        return [int(x) for x in out[:n]]

    def reused(self):
        return lib().tgohip_lease_reused(self.h)

    def len(self):
        return lib().tgohip_lease_len(self.h)

    def grow(self, n):
        check(lib().tgohip_lease_grow(self.h, n))

    def commit(self, ids):
        a = i32(ids or [0])
        check(lib().tgohip_lease_commit(self.h, ptr(a), len(ids)))

    def publish(self, written):
        lib().tgohip_lease_publish(self.h, written)
        return self.blocks()

    def release(self):
        lib().tgohip_lease_release(self.h)

    def free(self):
        if self.h:
            lib().tgohip_lease_free(self.h)
            self.h = None


class Pool:
    """prefix.Pool over the C ABI."""

    def __init__(self, block, blocks, scope=0):
        self.h = lib().tgohip_pool_new(block, blocks, scope)
        if not self.h:
            raise TgoError(EINVAL, last_error())
        self.leases = []

    def acquire(self, ids, session="", salt="", reserve=0):
        a = i32(ids or [0])
        out = ctypes.c_void_p()
        check(lib().tgohip_pool_acquire(self.h, ptr(a), len(ids), session.encode(), salt.encode(),
                                        reserve, ctypes.byref(out)))
        lease = Lease(out.value)
        self.leases.append(lease)
        return lease

    def stats(self):
        s = np.zeros(10, np.int64)
        lib().tgohip_pool_stats(self.h, ptr(s))
        keys = ("acquires", "hits", "reused", "prompt", "evictions", "publishes", "adoptions",
                "in_use", "cached", "free")
        return dict(zip(keys, (int(x) for x in s)))

    def close(self):
        for l in self.leases:
            l.free()
        self.leases = []
        if self.h:
            lib().tgohip_pool_free(self.h)
            self.h = None


def to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    sat = lib().tgohip_to_f16(ptr(x), ptr(out), x.size)
    return out, int(sat)


def quantize_int8(w):
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    q = np.empty(w.size, np.int8)
    s = np.empty((w.size + 31) // 32, np.uint16)
    lib().tgohip_quantize_int8(ptr(w), w.size, ptr(q), ptr(s))
    return q, s


def quantize_int4(w):
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    c = np.empty((w.size + 7) // 8, np.uint32)
    s = np.empty((w.size + 127) // 128, np.uint16)
    z = np.empty((w.size + 127) // 128, np.uint16)
    lib().tgohip_quantize_int4(ptr(w), w.size, ptr(c), ptr(s), ptr(z))
    return c, s, z


# ---------------------------------------------------------------------------
# device context
# ---------------------------------------------------------------------------

class SafeTensors:
    """safetensors.File (safetensors/safetensors.go): a validated header, planes on demand."""

    def __init__(self, path):
        self.h = lib().tgohip_st_open(os.fsencode(path))
        if not self.h:
            raise TgoError(EINVAL, last_error())

    def close(self):
        if self.h:
            lib().tgohip_st_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def entries(self):
        """-> {name: (dtype, shape tuple, begin, end)} in name order."""
        out = {}
        for i in range(lib().tgohip_st_count(self.h)):
            nm, dt = ctypes.c_char_p(), ctypes.c_char_p()
            rank = ctypes.c_int()
            shape = np.zeros(8, np.int64)
            b, e = ctypes.c_int64(), ctypes.c_int64()
            check(lib().tgohip_st_entry(self.h, i, ctypes.byref(nm), ctypes.byref(dt),
                                        ctypes.byref(rank), ptr(shape), ctypes.byref(b),
                                        ctypes.byref(e)))
            out[nm.value.decode()] = (dt.value.decode(), tuple(int(x) for x in shape[:rank.value]),
                                      b.value, e.value)
        return out

    def read(self, name):
        ent = self.entries()
        n = ent[name][3] - ent[name][2] if name in ent else 0
        buf = np.zeros(max(n, 1), np.uint8)
        got = check(lib().tgohip_st_read(self.h, name.encode(), ptr(buf), n))
        return buf[:got].tobytes()


def set_safetensors_header_cap(nbytes):
    """Lowers the header-length cap (0 restores 100 MiB)."""
    lib().tgohip_st_set_max_header(nbytes)


class Repo:
    """safetensors.Repo (safetensors/repo.go): one model directory, single or sharded."""

    def __init__(self, path):
        self.h = lib().tgohip_repo_open(os.fsencode(path))
        if not self.h:
            raise TgoError(EINVAL, last_error())

    def close(self):
        if self.h:
            lib().tgohip_repo_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def has(self, name):
        return bool(lib().tgohip_repo_has(self.h, name.encode()))

    def plane(self, name, n, transpose=False, head_dim=0):
        """The loader's f32 plane of `name` (decode, transpose, head permutation)."""
        out = np.zeros(n, np.float32)
        check(lib().tgohip_repo_plane(self.h, name.encode(), int(transpose), head_dim, ptr(out), n))
        return out


class Context:
    """One device, one stream: accel.Device + Queue for the batched path."""

    def __init__(self, device=0):
        self.h = lib().tgohip_open(device)
        if not self.h:
            raise TgoError(EDEVICE, last_error())
        self.cfg = None

    def close(self):
        if self.h:
            lib().tgohip_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def stream(self):
        return lib().tgohip_stream(self.h)

    def set_stream(self, s):
        """Launch on stream handle `s` (0 is the default stream)."""
        check(lib().tgohip_set_stream(self.h, s))

    def use_own_stream(self):
        check(lib().tgohip_use_own_stream(self.h))

    def sync(self):
        check(lib().tgohip_sync(self.h))

    def set_cascade(self, min_sharers):
        """Prefix-shared attention for groups of at least min_sharers decode
        sequences whose page tables begin alike (0: off, the default)."""
        check(lib().tgohip_set_cascade(self.h, min_sharers))

    def set_precision(self, mode):
        check(lib().tgohip_set_precision(self.h, mode))

    # ---- model ----
    def config(self, layers, hidden, heads, kv_heads, head_dim, ffn, vocab, rms_eps, rope_theta,
               block):
        c = ModelCfg(layers, hidden, heads, kv_heads, head_dim, ffn, vocab, rms_eps, rope_theta,
                     block)
        check(lib().tgohip_config(self.h, ctypes.byref(c)))
        self.cfg = dict(layers=layers, hidden=hidden, heads=heads, kv_heads=kv_heads,
                        head_dim=head_dim, ffn=ffn, vocab=vocab, rms_eps=rms_eps,
                        rope_theta=rope_theta, block=block)

    def weight(self, port, form, K, N, plane, scales=None, zeros=None):
        check(lib().tgohip_weight(self.h, port.encode(), form, K, N, ptr(plane), ptr(scales),
                                  ptr(zeros)))

    def weight_f32(self, port, form, K, N, w):
        """tgohip_weight from an f32 [K,N] plane, quantized (I8, I4_TGO) on the device."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        assert w.size == K * N
        check(lib().tgohip_weight_f32(self.h, port.encode(), form, K, N, ptr(w)))

    def gain(self, port, g):
        g = np.ascontiguousarray(g, dtype=np.float32)
        check(lib().tgohip_gain(self.h, port.encode(), ptr(g), g.size))

    def load_qwen3(self, repo, form, tie=False):
        """weights.Load of every Qwen3 port from `repo`; returns the f16 saturation count."""
        sat = ctypes.c_int64()
        check(lib().tgohip_load_qwen3(self.h, repo.h, form, int(tie), ctypes.byref(sat)))
        return sat.value

    def synth_weights(self, seed, form, sigma):
        check(lib().tgohip_synth_weights(self.h, seed, form, sigma))

    def kv_alloc(self, positions):
        check(lib().tgohip_kv_alloc(self.h, positions))

    def kv_synth(self, seed, sigma, positions):
        check(lib().tgohip_kv_synth(self.h, seed, sigma, positions))

    def probe_peaks(self, read_bytes=2 << 30, reps=5):
        """(read GB/s, dense f16 MFMA TFLOP/s) this box reaches: tgohip_probe_peaks."""
        gbps, tflops = ctypes.c_double(), ctypes.c_double()
        check(lib().tgohip_probe_peaks(self.h, read_bytes, reps, ctypes.byref(gbps),
                                       ctypes.byref(tflops)))
        return gbps.value, tflops.value

    def set_profile(self, on, stride=1):
        """Time the attention launch of every `stride`-th layer (HIP events)."""
        check(lib().tgohip_set_profile(self.h, stride if on else 0))

    def set_profile_kernels(self, stride, kinds):
        """Time the launches of the kernel kinds named (PROF_*) in every stride-th layer."""
        mask = 0
        for k in kinds:
            mask |= 1 << k
        check(lib().tgohip_set_profile_kernels(self.h, stride, mask))

    def profile_read_kernel(self, kind):
        """-> (ms, algorithmic bytes, flops, launches) summed over the timed launches."""
        ms, by, fl, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_double(), ctypes.c_int64()
        check(lib().tgohip_profile_read_kernel(self.h, kind, ctypes.byref(ms), ctypes.byref(by),
                                               ctypes.byref(fl), ctypes.byref(n)))
        return ms.value, by.value, fl.value, n.value

    def profile_read(self):
        ms, by, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int64()
        check(lib().tgohip_profile_read(self.h, ctypes.byref(ms), ctypes.byref(by),
                                        ctypes.byref(n)))
        return ms.value, by.value, n.value

    def kv_pointers(self):
        k, v, n = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int()
        check(lib().tgohip_kv_pointers(self.h, ctypes.byref(k), ctypes.byref(v), ctypes.byref(n)))
        return k.value, v.value, n.value

    def step(self, st, pages, max_pages, want_logits=True, want_argmax=True):
        """Batch.step's device half (batch.go:384-437). st: ports (dict of arrays).
        posq, posk and slots may be None (absent) together: the device derives them."""
        keep = {k: (u32(v) if v is not None else None) for k, v in st.items()}
        pg = u32(pages)
        B = len(keep["lengths"])
        addr = lambda a: None if a is None else ptr(a).value
        c = BatchStepC(len(keep["ids"]), B, max_pages, *(addr(keep.get(n)) for n in (
            "ids", "posq", "posk", "slots", "lengths", "extents", "last")), ptr(pg).value)
        logits = np.zeros((B, self.cfg["vocab"]), np.float32) if want_logits else None
        am = np.zeros(B, np.int32) if want_argmax else None
        t = Timings()
        check(lib().tgohip_step(self.h, ctypes.byref(c), ptr(logits), ptr(am), ctypes.byref(t)))
        return logits, am, t

    # ---- op level ----
    def paged_attention(self, q, T, H, Hkv, k, v, capacity, lengths, extents, pages, max_pages,
                        block, scale, out, q_dtype=F32, out_dtype=F32, head_dim=128):
        lengths, extents, pages = u32(lengths), u32(extents), u32(pages)
        check(lib().tgohip_paged_attention(self.h, ptr(q), q_dtype, T, H, Hkv, head_dim, ptr(k),
                                           ptr(v), capacity, len(lengths), ptr(lengths),
                                           ptr(extents), ptr(pages), max_pages, block, scale,
                                           ptr(out), out_dtype))

    def paged_attention_replay(self, q, T, H, Hkv, k, v, capacity, lengths, extents, pages,
                               max_pages, block, scale, out, iters, q_dtype=F32, out_dtype=F32):
        lengths, extents, pages = u32(lengths), u32(extents), u32(pages)
        check(lib().tgohip_paged_attention_replay(self.h, ptr(q), q_dtype, T, H, Hkv, ptr(k),
                                                  ptr(v), capacity, len(lengths), ptr(lengths),
                                                  ptr(extents), ptr(pages), max_pages, block,
                                                  scale, ptr(out), out_dtype, iters))

    def weight_upload(self, form, K, N, plane, scales=None, zeros=None):
        h = ctypes.c_int()
        check(lib().tgohip_weight_upload(self.h, form, K, N, ptr(plane), ptr(scales), ptr(zeros),
                                         ctypes.byref(h)))
        return h.value

    def weight_upload_f32(self, form, K, N, w):
        """An op-level weight from an f32 [K,N] plane quantized (I8, I4_TGO) on the device."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        assert w.size == K * N
        h = ctypes.c_int()
        check(lib().tgohip_weight_upload_f32(self.h, form, K, N, ptr(w), ctypes.byref(h)))
        return h.value

    def weight_synth(self, form, K, N, seed, stream, sigma):
        h = ctypes.c_int()
        check(lib().tgohip_weight_synth(self.h, form, K, N, seed, stream, sigma, ctypes.byref(h)))
        return h.value

    def weight_free(self, handle):
        check(lib().tgohip_weight_free(self.h, handle))

    def linear(self, handle, x, M, y, x_dtype=F32, y_dtype=F32):
        check(lib().tgohip_linear(self.h, handle, ptr(x), x_dtype, M, ptr(y), y_dtype))

    def greedy(self, logits, B, V, ids, margins=None):
        """sample argmax (first strict maximum) and TopTwoMargin over device rows."""
        check(lib().tgohip_greedy(self.h, ptr(logits), B, V, ptr(ids), ptr(margins)))

    def step_margins(self, B):
        """TopTwoMargin of each member of the last step (float64, host)."""
        out = np.zeros(B, np.float64)
        check(lib().tgohip_step_margins(self.h, ptr(out), B))
        return out

    def linear_noalloc(self, handle, x, M, y, x_dtype=F32, y_dtype=F32):
        """linear with its split-K partials in the library's static workspace."""
        check(lib().tgohip_linear_noalloc(self.h, handle, ptr(x), x_dtype, M, ptr(y), y_dtype))

    def linear_workspace(self, handle, M, x_dtype=F32):
        """Bytes of split-K partials a linear call over M rows uses (0: unsplit)."""
        n = ctypes.c_size_t()
        check(lib().tgohip_linear_workspace(self.h, handle, x_dtype, M, ctypes.byref(n)))
        return n.value

    def dequant(self, handle, y):
        check(lib().tgohip_dequant(self.h, handle, ptr(y)))

    def dequant_f16(self, handle, y):
        check(lib().tgohip_dequant_f16(self.h, handle, ptr(y)))


class Scheduler:
    """tgo.Scheduler (scheduler.go:34-397) over the C ABI: Admit, Step, Feed, Finish, Evict."""

    def __init__(self, ctx, n, chunk=0, reserve=1, max_rows=0):
        self.ctx = ctx
        self.n = n
        self.h = lib().tgohip_sched_new(ctx.h, n, chunk, reserve, max_rows)
        if not self.h:
            raise TgoError(EINVAL, last_error())

    def admit(self, prompt, reserve=0):
        a = i32(prompt or [0])
        return check(lib().tgohip_sched_admit(self.h, ptr(a), len(prompt), reserve))

    def admit_prefilled(self, prompt, feed, reserve=0):
        a = i32(prompt or [0])
        return check(lib().tgohip_sched_admit_prefilled(self.h, ptr(a), len(prompt), reserve,
                                                        feed))

    def prefilling(self):
        return lib().tgohip_sched_prefilling(self.h)

    def live(self):
        return lib().tgohip_sched_live(self.h)

    def last_step(self):
        """The ports of the last step: (dict of arrays, pages, max_pages)."""
        r, b, mp = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        L = lib()
        check(L.tgohip_sched_last_step(self.h, ctypes.byref(r), ctypes.byref(b),
                                       ctypes.byref(mp), *([None] * 8)))
        cfg = self.ctx.cfg
        rows, B, maxp = r.value, b.value, mp.value
        st = dict(ids=np.zeros(rows, np.uint32), posq=np.zeros(rows * cfg["heads"], np.uint32),
                  posk=np.zeros(rows * cfg["kv_heads"], np.uint32),
                  slots=np.zeros(rows, np.uint32), lengths=np.zeros(B, np.uint32),
                  extents=np.zeros(B, np.uint32), last=np.zeros(B, np.uint32))
        pages = np.zeros(B * maxp, np.uint32)
        L.tgohip_sched_last_step(self.h, ctypes.byref(r), ctypes.byref(b), ctypes.byref(mp),
                                 ptr(st["ids"]), ptr(st["posq"]), ptr(st["posk"]),
                                 ptr(st["slots"]), ptr(st["lengths"]), ptr(st["extents"]),
                                 ptr(st["last"]), ptr(pages))
        return st, pages, maxp

    def finish(self, slot):
        check(lib().tgohip_sched_finish(self.h, slot))

    def evict(self):
        return lib().tgohip_sched_evict(self.h)

    def feed(self, slot, token):
        check(lib().tgohip_sched_feed(self.h, slot, token))

    def length(self, slot):
        return lib().tgohip_sched_length(self.h, slot)

    def step(self):
        """-> ([(slot, greedy token, done)], prefill_tokens, decodes, timings)."""
        s, t, d = (np.zeros(self.n, np.int32) for _ in range(3))
        pf, dc = ctypes.c_int32(), ctypes.c_int32()
        tm = Timings()
        n = check(lib().tgohip_sched_step(self.h, ptr(s), ptr(t), ptr(d), ctypes.byref(pf),
                                          ctypes.byref(dc), ctypes.byref(tm)))
        return [(int(s[i]), int(t[i]), bool(d[i])) for i in range(n)], pf.value, dc.value, tm

    # ---- overlap mode: submit the next step before the last is read back ----
    def set_overlap(self, on):
        check(lib().tgohip_sched_set_overlap(self.h, 1 if on else 0))

    def submit(self):
        """Enqueues the next step. -> ([(slot, done)], prefill_tokens, decodes); an empty
        list when there is nothing to step."""
        s, d = np.zeros(self.n, np.int32), np.zeros(self.n, np.int32)
        pf, dc = ctypes.c_int32(), ctypes.c_int32()
        n = check(lib().tgohip_sched_submit(self.h, ptr(s), ptr(d), ctypes.byref(pf),
                                            ctypes.byref(dc)))
        return [(int(s[i]), bool(d[i])) for i in range(n)], pf.value, dc.value

    def collect(self):
        """Waits for the oldest step in flight. -> ([(slot, greedy token, done)], timings)."""
        s, t, d = (np.zeros(self.n, np.int32) for _ in range(3))
        tm = Timings()
        n = check(lib().tgohip_sched_collect(self.h, ptr(s), ptr(t), ptr(d), ctypes.byref(tm)))
        return [(int(s[i]), int(t[i]), bool(d[i])) for i in range(n)], tm

    def close(self):
        if self.h:
            lib().tgohip_sched_free(self.h)
            self.h = None
