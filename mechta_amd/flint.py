"""Python mirror of the Flint KV path's C ABI (include/mechta_flint.h), over the same libmechta_kv.so.

Flint (flint.rs:12-32): 32 query heads, 4 KV heads of 128, sliding layers on a ring of 1024 rows with a 513-position
window, full layers on ctx rows, per-head attention sinks. Every compute call goes through the HIP library.
"""
import ctypes

from mechta_amd import F16, F32, K, V, MkvError, _dev, _ptr, lib as _mkv_lib

Q_HEADS, KV_HEADS, HEAD_DIM = 32, 4, 128
RING_SWA, WINDOW, BLOCK_MAX = 1024, 513, 512

# every symbol include/mechta_flint.h declares
SYMBOLS = ["mfl_create", "mfl_destroy", "mfl_set_stream", "mfl_sync", "mfl_rows", "mfl_rope_table", "mfl_rope",
           "mfl_append", "mfl_attend", "mfl_read_rows", "mfl_write_rows", "mfl_photo", "mfl_restore_photo"]

_done = False


def lib():
    global _done
    L = _mkv_lib()
    if not _done:
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        sig = {
            "mfl_create": ([ctypes.POINTER(P), I, I, I, P, P], I),
            "mfl_destroy": ([P], I),
            "mfl_set_stream": ([P, P], I),
            "mfl_sync": ([P], I),
            "mfl_rows": ([P, I, ctypes.POINTER(I)], I),
            "mfl_rope_table": ([I, F, P], I),
            "mfl_rope": ([P, I, I, P, P, P], I),
            "mfl_append": ([P, I, I, I, P, P], I),
            "mfl_attend": ([P, I, I, I, P, P, P], I),
            "mfl_read_rows": ([P, I, I, I, I, P], I),
            "mfl_write_rows": ([P, I, I, I, I, P], I),
            "mfl_photo": ([P], I),
            "mfl_restore_photo": ([P], I),
        }
        for name, (args, res) in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _done = True
    return L


def _check(rc):
    if rc != 0:
        raise MkvError(rc, lib().mkv_last_error().decode())


def rope_table(pos, base=10000.0):
    """rope_table(pos, base) of flint.rs:61-68, computed by the library's host code: 128 floats."""
    buf = (ctypes.c_float * HEAD_DIM)()
    _check(lib().mfl_rope_table(int(pos), float(base), buf))
    return list(buf)


class FlintStore:
    """K/V of `layers` Flint layers; sliding[l] selects the 1024-row ring and the 513-position window.

    append = kv_write / kv_write_n, attend = attn_fd + attn_fd_merge (one token) or attn_pf (a block), rope =
    rope_neox(_n), read_rows / write_rows = the reference's row layout (roots), photo / restore_photo = the ring photo.
    """

    def __init__(self, layers, ctx, fmt=F32, sliding=None, stream=None):
        import torch
        self.layers, self.ctx, self.fmt = layers, ctx, fmt
        self.sliding = [bool(x) for x in (sliding if sliding is not None else [False] * layers)]
        mask = (ctypes.c_ubyte * layers)(*[1 if s else 0 for s in self.sliding])
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        self._h = ctypes.c_void_p()
        _check(lib().mfl_create(ctypes.byref(self._h), layers, ctx, fmt, mask, ctypes.c_void_p(stream)))

    def close(self):
        if self._h:
            _check(lib().mfl_destroy(self._h))
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        """The store's mfl_t* (ctypes.c_void_p), for a caller that calls the C ABI through lib() directly."""
        return self._h

    def set_stream(self, stream):
        """Later calls enqueue on `stream` (a torch.cuda.Stream), e.g. torch's stream while capturing a graph."""
        _check(lib().mfl_set_stream(self._h, ctypes.c_void_p(stream.cuda_stream)))

    def sync(self):
        _check(lib().mfl_sync(self._h))

    def rows(self, layer):
        r = ctypes.c_int()
        _check(lib().mfl_rows(self._h, layer, ctypes.byref(r)))
        return r.value

    def rope(self, x, tab, out=None):
        """NEOX RoPE of x [ntok][heads][128] by table rows tab [ntok][128] (device tensors)."""
        import torch
        ntok = tab.shape[0]
        heads = x.numel() // (ntok * HEAD_DIM)
        if out is None:
            out = torch.empty_like(x)
        _check(lib().mfl_rope(self._h, ntok, heads, _dev(x, ntok * heads * HEAD_DIM, "x"),
                              _dev(tab, ntok * HEAD_DIM, "tab"), _dev(out, ntok * heads * HEAD_DIM, "out")))
        return out

    def append(self, layer, pos0, k, v):
        ntok = k.numel() // (KV_HEADS * HEAD_DIM)
        n = ntok * KV_HEADS * HEAD_DIM
        _check(lib().mfl_append(self._h, layer, pos0, ntok, _dev(k, n, "k"), _dev(v, n, "v")))

    def attend(self, layer, pos0, q, sinks=None, out=None):
        import torch
        ntok = q.numel() // (Q_HEADS * HEAD_DIM)
        if out is None:
            out = torch.empty((ntok, Q_HEADS, HEAD_DIM), dtype=torch.float32, device="cuda")
        s = None if sinks is None else _dev(sinks, Q_HEADS, "sinks")
        _check(lib().mfl_attend(self._h, layer, pos0, ntok, _dev(q, ntok * Q_HEADS * HEAD_DIM, "q"), s,
                                _dev(out, ntok * Q_HEADS * HEAD_DIM, "out")))
        return out

    def read_rows(self, layer, which, r0, r1, out=None):
        """Rows [r0, r1) of K or V in the reference layout [row][4][128] (int16 bit patterns for f16)."""
        import torch
        dt = torch.int16 if self.fmt == F16 else torch.float32
        if out is None:
            out = torch.empty((r1 - r0, KV_HEADS, HEAD_DIM), dtype=dt, device="cuda")
        _check(lib().mfl_read_rows(self._h, layer, which, r0, r1, _ptr(out)))
        return out

    def write_rows(self, layer, which, r0, r1, rows):
        _check(lib().mfl_write_rows(self._h, layer, which, r0, r1, _ptr(rows)))

    def photo(self):
        _check(lib().mfl_photo(self._h))

    def restore_photo(self):
        _check(lib().mfl_restore_photo(self._h))


__all__ = ["FlintStore", "rope_table", "SYMBOLS", "F16", "F32", "K", "V"]
