"""mechta_amd: MI355X-native KV-cache path of mechta (f16/f32 KV store, append with rollback, split-K flash decode,
causal prefill flash attention, prefix-cache snapshot), behind the C ABI of include/mechta_kv.h.

This module is the Python host mirror of that ABI (ctypes over mechta_amd/lib/libmechta_kv.so). Device buffers are
torch tensors used as plain HBM allocations; every compute call goes through the HIP library, and a missing or
unloadable library raises instead of computing anything another way.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmechta_kv.so")

F16, F32 = 0, 1
K, V = 0, 1
KV_HEADS, Q_HEADS, HEAD_DIM = 2, 16, 256
CTX_MIN, CTX_MAX = 4096, 262144
PREFILL_MAX = 512

E_ARG, E_CTX, E_POS, E_LAYER, E_SIZE, E_HIP, E_NOMEM, E_FMT, E_IO = -1, -2, -3, -4, -5, -6, -7, -8, -9

# every symbol include/mechta_kv.h declares
SYMBOLS = ["mkv_create", "mkv_destroy", "mkv_set_stream", "mkv_sync", "mkv_last_error", "mkv_info", "mkv_len",
           "mkv_append", "mkv_set_len", "mkv_decode", "mkv_append_decode", "mkv_prefill", "mkv_snapshot_bytes",
           "mkv_snapshot", "mkv_restore", "mkv_read_rows", "mkv_write_rows", "mkv_trace", "mkv_trace_read",
           "mkv_rope_table", "mkv_root_key", "mkv_root_save", "mkv_root_wait", "mkv_root_info", "mkv_root_load",
           "mkv_rope_table_dev", "mkv_qk_norm_rope", "mkv_buffer_bytes", "mkv_store_bytes",
           "mkv_append_decode_noalloc", "mkv_decode_g16", "mkv_append_decode_g16", "mkv_noalloc_scratch_bytes",
           "mkv_root_path", "mkv_root_prune", "mkv_root_touch"]
SPAN_KV_WRITE, SPAN_CORE, SPAN_MERGE = 0, 1, 2


class MkvError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None


def lib():
    """Loads libmechta_kv.so (raises if it was not built: run __graft_entry__.build())."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with python -c 'import __graft_entry__ as g; "
                               f"g.build()'")
        L = ctypes.CDLL(LIB_PATH)
        P, I, F, S, U64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_uint64
        sig = {
            "mkv_create": ([ctypes.POINTER(P), I, I, I, P], I),
            "mkv_destroy": ([P], I),
            "mkv_set_stream": ([P, P], I),
            "mkv_sync": ([P], I),
            "mkv_last_error": ([], ctypes.c_char_p),
            "mkv_info": ([P, ctypes.POINTER(I), ctypes.POINTER(I), ctypes.POINTER(I)], I),
            "mkv_len": ([P, I, ctypes.POINTER(I)], I),
            "mkv_append": ([P, I, I, I, P, P, P], I),
            "mkv_set_len": ([P, I], I),
            "mkv_decode": ([P, I, P, I, I, I, F, P, P], I),
            "mkv_append_decode": ([P, I, I, I, P, P, P, P, I, F, P, P], I),
            "mkv_append_decode_noalloc": ([P, I, I, I, P, P, P, P, I, F, P, P], I),
            "mkv_decode_g16": ([P, I, P, I, I, I, F, P, P], I),
            "mkv_append_decode_g16": ([P, I, I, I, P, P, P, P, I, F, P, P], I),
            "mkv_prefill": ([P, I, P, I, I, I, F, P, P], I),
            "mkv_snapshot_bytes": ([P, I], S),
            "mkv_snapshot": ([P, I, P, S], I),
            "mkv_restore": ([P, I, P, S], I),
            "mkv_read_rows": ([P, I, I, I, I, P], I),
            "mkv_write_rows": ([P, I, I, I, I, P], I),
            "mkv_trace": ([P, I], I),
            "mkv_trace_read": ([P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_long)], I),
            "mkv_rope_table": ([I, P], I),
            "mkv_root_key": ([P, S], U64),
            "mkv_root_save": ([P, ctypes.c_char_p, I, P, I, P, P, P, P, I], I),
            "mkv_root_wait": ([P], I),
            "mkv_root_info": ([ctypes.c_char_p, ctypes.POINTER(I), ctypes.POINTER(I), ctypes.POINTER(I),
                               ctypes.POINTER(U64), P, P, I], I),
            "mkv_root_load": ([P, ctypes.c_char_p, P, P, P], I),
            "mkv_rope_table_dev": ([P, I, ctypes.POINTER(P)], I),
            "mkv_qk_norm_rope": ([P, I, I, P, P, P, P, F, P, P], I),
            "mkv_buffer_bytes": ([I, I], S),
            "mkv_store_bytes": ([I, I, I], S),
            "mkv_noalloc_scratch_bytes": ([], S),
            "mkv_root_path": ([ctypes.c_char_p, S, ctypes.c_char_p, I, ctypes.c_char_p, P, S], I),
            "mkv_root_prune": ([ctypes.c_char_p, I, I], I),
            "mkv_root_touch": ([ctypes.c_char_p], I),
        }
        for name, (args, res) in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def buffer_bytes(ctx, fmt):
    """Bytes of one K or V cache of one layer (the reference's KvFormat::buffer_bytes_for)."""
    return lib().mkv_buffer_bytes(ctx, fmt)


def store_bytes(layers, ctx, fmt):
    """Device bytes mkv_create allocates for such a store (0 if it would refuse the arguments)."""
    return lib().mkv_store_bytes(layers, ctx, fmt)


def _check(rc):
    if rc != 0:
        raise MkvError(rc, lib().mkv_last_error().decode())


def _ptr(t):
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def _dev(t, n, name, f16=False):
    """Checks a torch tensor argument: on a GPU, float32 (float16 with f16), contiguous, at least n elements."""
    import torch
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor")
    want = torch.float16 if f16 else torch.float32
    if t.dtype != want or not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous {str(want).split('.')[-1]}")
    if t.numel() < n:
        raise ValueError(f"{name} holds {t.numel()} values, {n} needed")
    return _ptr(t)


def rope_table(pos):
    """rope_table(pos) of the reference (engine.rs:108-114), computed by the library's host code: 64 floats."""
    buf = (ctypes.c_float * 64)()
    _check(lib().mkv_rope_table(int(pos), buf))
    return list(buf)


def root_key(tokens):
    """FNV-1a 64 of the tokens' little-endian bytes (root_key, session.rs:62-66), computed by the library."""
    import numpy as np
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    return lib().mkv_root_key(t.ctypes.data_as(ctypes.c_void_p), t.size)


def root_path(dir, fmt, model_path, tokens):
    """File name of a root (root_file, session.rs:68-73): <dir>/root-<f16|f32>-<model key>-<token key>.bin."""
    import numpy as np
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    buf = ctypes.create_string_buffer(4096)
    n = lib().mkv_root_path(buf, len(buf), os.fsencode(dir), fmt, os.fsencode(model_path),
                            t.ctypes.data_as(ctypes.c_void_p), t.size)
    _check(n if n < 0 else 0)
    return os.fsdecode(buf.value)


def root_prune(dir, fmt, keep=6):
    """Keeps the `keep` most recently modified root files of the format in `dir` (prune_roots, session.rs:75-84);
    returns how many it removed."""
    n = lib().mkv_root_prune(os.fsencode(dir), fmt, keep)
    _check(n if n < 0 else 0)
    return n


def root_touch(path):
    """Marks a root file as just used (touch, session.rs:86-88)."""
    _check(lib().mkv_root_touch(os.fsencode(path)))


ROOT_MIN = 2048  # session.rs:90: a root only for a system prompt of at least this many tokens


def root_info(path):
    """Counts of a root file: dict(p, ns, nk, kv_words, ssm_words, conv_words)."""
    p, ns, nk, kw = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_uint64()
    _check(lib().mkv_root_info(os.fsencode(path), ctypes.byref(p), ctypes.byref(ns), ctypes.byref(nk),
                               ctypes.byref(kw), None, None, 0))
    sw = (ctypes.c_uint64 * max(ns.value, 1))()
    cw = (ctypes.c_uint64 * max(ns.value, 1))()
    _check(lib().mkv_root_info(os.fsencode(path), None, None, None, None, sw, cw, ns.value))
    return dict(p=p.value, ns=ns.value, nk=nk.value, kv_words=kw.value, ssm_words=list(sw)[:ns.value],
                conv_words=list(cw)[:ns.value])


def _device_view(addr, n):
    """A float32 torch tensor over n floats of device memory the library owns (no copy, no ownership)."""
    import torch

    class _Mem:  # __cuda_array_interface__ provider
        __cuda_array_interface__ = {"shape": (n,), "typestr": "<f4", "data": (addr, False), "version": 2}

    return torch.as_tensor(_Mem(), device="cuda")


def _ptr_array(arrays):
    return (ctypes.c_void_p * max(len(arrays), 1))(*[a.ctypes.data for a in arrays])


def _pinned(t, who):
    if t.device.type != "cpu" or not t.is_pinned():
        raise ValueError(f"{who}: the host buffer must be pinned host memory (torch pin_memory=True / hipHostMalloc)")


class KvStore:
    """The KV store of `layers` full-attention layers (K and V, 2 KV heads x 256, `ctx` positions, f16 or f32).

    Mirrors the KV-cache part of the reference's Engine: append = kv_rope2 + kv_copy, decode = attn_fd / attn_dmx2 +
    attn_fd_combine (+ attn_gate), prefill = attn_fa_mx + attn_fd_combine, snapshot/restore = read_root / write_root
    (KV part). All tensors are torch device tensors; calls are ordered on `stream` (default: torch's current stream).
    """

    def __init__(self, layers, ctx, fmt=F16, stream=None):
        import torch
        self.layers, self.ctx, self.fmt = layers, ctx, fmt
        s = stream if stream is not None else torch.cuda.current_stream()
        self._stream = s
        h = ctypes.c_void_p()
        _check(lib().mkv_create(ctypes.byref(h), layers, ctx, fmt, ctypes.c_void_p(s.cuda_stream)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            lib().mkv_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def handle(self):
        """The store's mkv_t* (ctypes.c_void_p), for a caller that calls the C ABI through lib() directly (bench.py's
        step loops: no Python argument checks between launches)."""
        return self._h

    def set_stream(self, stream):
        self._stream = stream
        _check(lib().mkv_set_stream(self._h, ctypes.c_void_p(stream.cuda_stream)))

    def sync(self):
        _check(lib().mkv_sync(self._h))
        self._restore_src = None  # the copy out of it has landed

    def length(self, layer=0):
        n = ctypes.c_int()
        _check(lib().mkv_len(self._h, layer, ctypes.byref(n)))
        return n.value

    def append(self, layer, pos, k_normed, v, rope_tab):
        ntok = k_normed.numel() // (KV_HEADS * HEAD_DIM)
        _check(lib().mkv_append(self._h, layer, pos, ntok, _dev(k_normed, ntok * 512, "k_normed"),
                                _dev(v, ntok * 512, "v"), _dev(rope_tab, ntok * 64, "rope_tab")))

    def set_len(self, n):
        _check(lib().mkv_set_len(self._h, n))

    def decode(self, layer, q, n, start=0, scale=1.0 / 16, out=None, gate_src=None, f16_out=False):
        """f16_out: the gated attention as float16 (mkv_decode_g16, the reference's attn_gate16); needs gate_src."""
        import torch
        ntok = q.numel() // (Q_HEADS * HEAD_DIM)
        if out is None:
            out = torch.empty((ntok, Q_HEADS, HEAD_DIM), dtype=torch.float16 if f16_out else torch.float32,
                              device=q.device)
        g = None if gate_src is None else _dev(gate_src, ntok * Q_HEADS * 512, "gate_src")
        fn = lib().mkv_decode_g16 if f16_out else lib().mkv_decode
        _check(fn(self._h, layer, _dev(q, ntok * 4096, "q"), ntok, n, start, scale,
                  _dev(out, ntok * 4096, "out", f16_out), g))
        return out

    def append_decode(self, layer, n, k_normed, v, rope_tab, q, start=0, scale=1.0 / 16, out=None, gate_src=None,
                      f16_out=False):
        """f16_out as decode (mkv_append_decode_g16)."""
        import torch
        ntok = q.numel() // (Q_HEADS * HEAD_DIM)
        if out is None:
            out = torch.empty((ntok, Q_HEADS, HEAD_DIM), dtype=torch.float16 if f16_out else torch.float32,
                              device=q.device)
        g = None if gate_src is None else _dev(gate_src, ntok * Q_HEADS * 512, "gate_src")
        fn = lib().mkv_append_decode_g16 if f16_out else lib().mkv_append_decode
        _check(fn(self._h, layer, n, ntok, _dev(k_normed, ntok * 512, "k_normed"), _dev(v, ntok * 512, "v"),
                  _dev(rope_tab, ntok * 64, "rope_tab"), _dev(q, ntok * 4096, "q"), start, scale,
                  _dev(out, ntok * 4096, "out", f16_out), g))
        return out

    def prefill(self, layer, q, n, start=0, scale=1.0 / 16, out=None, gate_src=None):
        import torch
        T = q.numel() // (Q_HEADS * HEAD_DIM)
        if out is None:
            out = torch.empty((T, Q_HEADS, HEAD_DIM), dtype=torch.float32, device=q.device)
        g = None if gate_src is None else _dev(gate_src, T * Q_HEADS * 512, "gate_src")
        _check(lib().mkv_prefill(self._h, layer, _dev(q, T * 4096, "q"), T, n, start, scale,
                                 _dev(out, T * 4096, "out"), g))
        return out

    def trace(self, enable=True):
        _check(lib().mkv_trace(self._h, 1 if enable else 0))

    def trace_read(self):
        """{span: (total kernel ms, launches)} for kv_write, core, merge since tracing started (waits)."""
        ms = (ctypes.c_double * 3)()
        cnt = (ctypes.c_long * 3)()
        _check(lib().mkv_trace_read(self._h, ms, cnt))
        return {name: (ms[i], cnt[i]) for i, name in enumerate(("kv_write", "core", "merge"))}

    def snapshot_bytes(self, p):
        return lib().mkv_snapshot_bytes(self._h, p)

    def snapshot(self, p, host=None):
        """KV of positions [0, p) of every layer into pinned host memory (a uint8 tensor)."""
        import torch
        nb = self.snapshot_bytes(p)
        if host is None:
            host = torch.empty(nb, dtype=torch.uint8, pin_memory=True)
        _pinned(host, "snapshot")
        _check(lib().mkv_snapshot(self._h, p, _ptr(host), host.numel() * host.element_size()))
        return host

    def restore(self, p, host):
        """Positions [0, p) of every layer from a snapshot in pinned host memory. The copy is only enqueued: the
        store keeps a reference to `host` until the next sync() (do not write into it before then)."""
        _pinned(host, "restore")
        _check(lib().mkv_restore(self._h, p, _ptr(host), host.numel() * host.element_size()))
        self._restore_src = host

    def read_rows(self, layer, which, p0, p1, out=None):
        """Positions [p0, p1) of K or V in the reference layout [pos][2][256] (int16 bit patterns for f16)."""
        import torch
        dt = torch.int16 if self.fmt == F16 else torch.float32
        if out is None:
            out = torch.empty((p1 - p0, KV_HEADS, HEAD_DIM), dtype=dt, device="cuda")
        _check(lib().mkv_read_rows(self._h, layer, which, p0, p1, _ptr(out)))
        return out

    def write_rows(self, layer, which, p0, p1, rows):
        _check(lib().mkv_write_rows(self._h, layer, which, p0, p1, _ptr(rows)))

    def rope_table_dev(self, pos, ntok):
        """Rows pos .. pos + ntok - 1 of the store's device RoPE table, as a float32 device tensor view [ntok][64]."""
        import torch
        ptr = ctypes.c_void_p()
        _check(lib().mkv_rope_table_dev(self._h, pos, ctypes.byref(ptr)))
        if not hasattr(self, "_rope_view"):
            # a tensor over the whole table (its allocation belongs to the store): rows are slices of it
            base = ctypes.c_void_p()
            _check(lib().mkv_rope_table_dev(self._h, 0, ctypes.byref(base)))
            self._rope_base = base.value
            self._rope_view = _device_view(base.value, self.ctx * 64)
        off = (ptr.value - self._rope_base) // 4
        return self._rope_view[off:off + ntok * 64].view(ntok, 64)

    def qk_norm_rope(self, pos, qf, kb, q_norm_w, k_norm_w, eps=1e-6, q_out=None, kn_out=None):
        """q/k producer: (rope2(rmsnorm(q)) [ntok][16][256], rmsnorm(k) [ntok][2][256]) from qf [ntok][16][512]
        and kb [ntok][2][256] (device tensors)."""
        import torch
        ntok = qf.numel() // (Q_HEADS * 512)
        if q_out is None:
            q_out = torch.empty((ntok, Q_HEADS, HEAD_DIM), dtype=torch.float32, device=qf.device)
        if kn_out is None:
            kn_out = torch.empty((ntok, KV_HEADS, HEAD_DIM), dtype=torch.float32, device=qf.device)
        _check(lib().mkv_qk_norm_rope(self._h, pos, ntok, _dev(qf, ntok * 8192, "qf"), _dev(kb, ntok * 512, "kb"),
                                      _dev(q_norm_w, 256, "q_norm_w"), _dev(k_norm_w, 256, "k_norm_w"), eps,
                                      _dev(q_out, ntok * 4096, "q_out"), _dev(kn_out, ntok * 512, "kn_out")))
        return q_out, kn_out

    def root_save(self, path, p, tokens, ssm=(), conv=(), background=False):
        """Writes a root file (the reference's container) of positions [0, p) of every layer, the p tokens and the
        caller's state vectors (float32 arrays, ssm[i] with conv[i])."""
        import numpy as np
        tok = np.ascontiguousarray(tokens, dtype=np.uint32)
        assert tok.size == p and len(ssm) == len(conv)
        ssm = [np.ascontiguousarray(a, dtype=np.float32) for a in ssm]
        conv = [np.ascontiguousarray(a, dtype=np.float32) for a in conv]
        sw = (ctypes.c_uint64 * max(len(ssm), 1))(*[a.size for a in ssm])
        cw = (ctypes.c_uint64 * max(len(conv), 1))(*[a.size for a in conv])
        _check(lib().mkv_root_save(self._h, os.fsencode(path), p, tok.ctypes.data_as(ctypes.c_void_p), len(ssm),
                                   _ptr_array(ssm), sw, _ptr_array(conv), cw, 1 if background else 0))

    def root_wait(self):
        _check(lib().mkv_root_wait(self._h))

    def root_load(self, path):
        """Puts a root file into the store; returns (p, tokens, ssm list, conv list) of the file."""
        import numpy as np
        info = root_info(path)
        tok = np.empty(info["p"], np.uint32)
        ssm = [np.empty(n, np.float32) for n in info["ssm_words"]]
        conv = [np.empty(n, np.float32) for n in info["conv_words"]]
        _check(lib().mkv_root_load(self._h, os.fsencode(path), tok.ctypes.data_as(ctypes.c_void_p),
                                   _ptr_array(ssm), _ptr_array(conv)))
        return info["p"], tok, ssm, conv
