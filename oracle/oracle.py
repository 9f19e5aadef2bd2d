"""ctypes wrapper of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the checker of the HIP
path. Caches handled here use the reference's position-major layout: [pos][kvh=2][256] per layer, f16 caches as
uint16 bit patterns (see mkv_oracle.h).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libmkv_oracle.so")

KVH, H, D = 2, 16, 256
ROW = KVH * D

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from oracle import build as _b  # noqa: WPS433 (build on first use, CPU only)
            _b.build()
        _lib = ctypes.CDLL(LIB_PATH)
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        _lib.orc_f32_to_f16.argtypes = [F]
        _lib.orc_f32_to_f16.restype = ctypes.c_uint16
        _lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.orc_f16_to_f32.restype = F
        _lib.orc_f32_to_f16_n.argtypes = [P, P, ctypes.c_int64]
        _lib.orc_rope_table.argtypes = [ctypes.c_int32, P]
        _lib.orc_append.argtypes = [I, P, P, I, I, P, P, P]
        _lib.orc_attn_fd.argtypes = [I, P, P, P, I, I, I, F, I, P]
        _lib.orc_attn_dmx.argtypes = [P, P, P, I, I, F, I, P]
        _lib.orc_attn_fa_mx.argtypes = [P, P, P, I, I, I, F, I, P, I, P]
        _lib.orc_attn_fa_f32.argtypes = [P, P, P, I, I, I, F, P, I, P]
        _lib.orc_attn_fd4.argtypes = [I, P, P, P, I, I, F, I, P]
        _lib.orc_gate.argtypes = [P, P, I, P]
        _lib.orc_gate16.argtypes = [P, P, I, P]
        _lib.orc_rmsnorm_rows.argtypes = [P, I, I, P, F, P]
        _lib.orc_qk_norm_rope.argtypes = [P, P, I, P, P, F, P, P, P]
        _lib.orc_threads.restype = I
        _lib.orc_fl_rope_table.argtypes = [I, F, P]
        _lib.orc_fl_rope.argtypes = [I, I, P, P, P]
        _lib.orc_fl_kv_write.argtypes = [I, P, P, I, I, I, P, P]
        _lib.orc_fl_attn_fd.argtypes = [I, P, P, I, P, I, I, P, P]
        _lib.orc_fl_attn_pf.argtypes = [I, P, P, I, P, I, I, I, P, P]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    a = np.ascontiguousarray(a, dtype=dt)
    return a


def f32_to_f16_bits(x):
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_p(x), _p(y), x.size)
    return y


def f16_bits_to_f32(h):
    return np.ascontiguousarray(h, np.uint16).view(np.float16).astype(np.float32)


def rope_table(pos):
    t = np.empty(64, np.float32)
    lib().orc_rope_table(int(pos), _p(t))
    return t


def rope_tables(pos, ntok):
    return np.stack([rope_table(pos + t) for t in range(ntok)])


def new_cache(ctx, fmt):
    """One layer's K or V cache in the reference layout, zero filled (wgpu zero-initialises buffers)."""
    return np.zeros((ctx, KVH, D), np.uint16 if fmt == 0 else np.float32)


def append(fmt, kc, vc, pos, kn, v, tab):
    kn = _c(kn, np.float32).reshape(-1, KVH, D)
    ntok = kn.shape[0]
    v = _c(v, np.float32).reshape(ntok, ROW)
    tab = _c(tab, np.float32).reshape(ntok, 64)
    assert kc.flags.c_contiguous and vc.flags.c_contiguous
    assert pos + ntok <= kc.shape[0]
    lib().orc_append(int(fmt), _p(kc), _p(vc), int(pos), ntok, _p(kn), _p(v), _p(tab))


def attn_fd(fmt, kc, vc, q, n, start=0, scale=1.0 / 16, bb=128):
    q = _c(q, np.float32).reshape(-1, H, D)
    ntok = q.shape[0]
    assert n + ntok - 1 <= kc.shape[0]
    out = np.empty((ntok, H, D), np.float32)
    lib().orc_attn_fd(int(fmt), _p(kc), _p(vc), _p(q), ntok, int(n), int(start), float(scale), int(bb), _p(out))
    return out


def attn_dmx(kc, vc, q, n, scale=1.0 / 16, ch=2048):
    q = _c(q, np.float32).reshape(-1, H, D)
    ntok = q.shape[0]
    assert 1 <= ntok <= 4 and n + ntok - 1 <= kc.shape[0]
    assert kc.dtype == np.uint16
    out = np.empty((ntok, H, D), np.float32)
    lib().orc_attn_dmx(_p(kc), _p(vc), _p(q), ntok, int(n), float(scale), int(ch), _p(out))
    return out


def attn_fa_mx(kc, vc, q, n, start=0, scale=1.0 / 16, ch=2048, sel=None):
    q = _c(q, np.float32).reshape(-1, H, D)
    T = q.shape[0]
    assert kc.dtype == np.uint16 and n + T - 1 <= kc.shape[0]
    if sel is None:
        sel = np.arange(T, dtype=np.int32)
    sel = _c(sel, np.int32)
    out = np.empty((len(sel), H, D), np.float32)
    lib().orc_attn_fa_mx(_p(kc), _p(vc), _p(q), T, int(n), int(start), float(scale), int(ch), _p(sel), len(sel),
                         _p(out))
    return out


def attn_fa_f32(kc, vc, q, n, start=0, scale=1.0 / 16, sel=None):
    q = _c(q, np.float32).reshape(-1, H, D)
    T = q.shape[0]
    assert kc.dtype == np.float32 and n + T - 1 <= kc.shape[0]
    if sel is None:
        sel = np.arange(T, dtype=np.int32)
    sel = _c(sel, np.int32)
    out = np.empty((len(sel), H, D), np.float32)
    lib().orc_attn_fa_f32(_p(kc), _p(vc), _p(q), T, int(n), int(start), float(scale), _p(sel), len(sel), _p(out))
    return out


def attn_fd4(fmt, kc, vc, q, n, scale=1.0 / 16, bl=64):
    """Small-block prefill (attn_fd4, ops.wgsl:694-778): token t of the block sees [0, n + t)."""
    q = _c(q, np.float32).reshape(-1, H, D)
    T = q.shape[0]
    assert n + T - 1 <= kc.shape[0] and bl % 64 == 0
    out = np.empty((T, H, D), np.float32)
    lib().orc_attn_fd4(int(fmt), _p(kc), _p(vc), _p(q), T, int(n), float(scale), int(bl), _p(out))
    return out


def gate(att, qf):
    att = _c(att, np.float32).reshape(-1, H * D)
    ntok = att.shape[0]
    qf = _c(qf, np.float32).reshape(ntok, H * 512)
    out = np.empty_like(att)
    lib().orc_gate(_p(att), _p(qf), ntok, _p(out))
    return out


def gate16(att, qf):
    """attn_gate16: the gated attention as f16 bits (uint16), rounded to nearest even."""
    att = _c(att, np.float32).reshape(-1, H * D)
    ntok = att.shape[0]
    qf = _c(qf, np.float32).reshape(ntok, H * 512)
    out = np.empty(att.shape, np.uint16)
    lib().orc_gate16(_p(att), _p(qf), ntok, _p(out))
    return out


def rmsnorm_rows(x, w, eps=1e-6, step=256):
    """rmsnorm (ops.wgsl:27-57) of the 256-value rows of x (row r at flat offset r*step) with weight w."""
    x = _c(x, np.float32).reshape(-1)
    rows = (x.size - 256) // step + 1
    out = np.empty((rows, 256), np.float32)
    lib().orc_rmsnorm_rows(_p(x), rows, int(step), _p(_c(w, np.float32)), float(eps), _p(out))
    return out


def qk_norm_rope(qf, kb, q_w, k_w, tab, eps=1e-6):
    """q/k producer (quad.rs:113-115): (q normed + rotated [ntok][16][256], k normed [ntok][2][256])."""
    qf = _c(qf, np.float32).reshape(-1, 16, 512)
    ntok = qf.shape[0]
    kb = _c(kb, np.float32).reshape(ntok, 2, 256)
    q_out = np.empty((ntok, 16, 256), np.float32)
    kn_out = np.empty((ntok, 2, 256), np.float32)
    lib().orc_qk_norm_rope(_p(qf), _p(kb), ntok, _p(_c(q_w, np.float32)), _p(_c(k_w, np.float32)), float(eps),
                           _p(_c(tab, np.float32).reshape(ntok, 64)), _p(q_out), _p(kn_out))
    return q_out, kn_out


def threads():
    return lib().orc_threads()


# ---------------------------------------------------------------- Flint (flint_oracle.c) ----------------------------
# Flint caches: [ring][4 kvh][128] per layer (row = position % ring), f32 or f16 bit patterns.
FL_H, FL_KVH, FL_D = 32, 4, 128
FL_WINDOW, FL_RING = 513, 1024


def _pp(a):
    return None if a is None else _p(a)


def fl_rope_table(pos, base=10000.0):
    t = np.empty(FL_D, np.float32)
    lib().orc_fl_rope_table(pos, base, _p(t))
    return t


def fl_rope_tables(pos0, ntok, base=10000.0):
    return np.stack([fl_rope_table(pos0 + t, base) for t in range(ntok)])


def fl_rope(x, tabs):
    x = _c(x, np.float32)
    ntok = tabs.shape[0]
    heads = x.size // (ntok * FL_D)
    out = np.empty_like(x)
    lib().orc_fl_rope(ntok, heads, _p(x), _p(_c(tabs, np.float32)), _p(out))
    return out


def fl_new_cache(rows, fmt):
    return np.zeros((rows, FL_KVH, FL_D), np.uint16 if fmt == 0 else np.float32)


def fl_kv_write(fmt, kc, vc, pos0, k, v):
    k, v = _c(k, np.float32), _c(v, np.float32)
    n = k.size // (FL_KVH * FL_D)
    lib().orc_fl_kv_write(fmt, _p(kc), _p(vc), kc.shape[0], pos0, n, _p(k), _p(v))


def fl_window_lo(pos, win):
    return pos + 1 - win if win and pos + 1 > win else 0


def fl_attn_fd(fmt, kc, vc, q, pos, win, sinks):
    """One token at position `pos`: positions [lo, pos] as attn_fd + attn_fd_merge."""
    q = _c(q, np.float32)
    lo = fl_window_lo(pos, win)
    out = np.empty((FL_H, FL_D), np.float32)
    s = None if sinks is None else _c(sinks, np.float32)
    lib().orc_fl_attn_fd(fmt, _p(kc), _p(vc), kc.shape[0], _p(q), lo, pos + 1 - lo, _pp(s), _p(out))
    return out


def fl_attn_pf(fmt, kc, vc, q, pos0, win, sinks):
    """Block of n tokens at pos0 .. pos0 + n - 1 as attn_pf."""
    q = _c(q, np.float32).reshape(-1, FL_H, FL_D)
    out = np.empty_like(q)
    s = None if sinks is None else _c(sinks, np.float32)
    lib().orc_fl_attn_pf(fmt, _p(kc), _p(vc), kc.shape[0], _p(q), pos0, q.shape[0], win, _pp(s), _p(out))
    return out
