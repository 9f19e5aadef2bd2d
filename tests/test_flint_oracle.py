"""CPU tests of the Flint part of the oracle (oracle/flint_oracle.c) against independent computations, and of the
Flint C ABI's host side (exported symbols, the host RoPE table). No GPU.

The reference has no tests or fixtures of its own for these kernels (flint_attn.wgsl); each restated function is
pinned here by float64 arithmetic, closed forms and invariants chosen so that a wrong index, sign, mask bound or
sink treatment fails."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import mechta_amd as mk
from mechta_amd import flint as mf
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mechta_flint.h")
H, KVH, D = 32, 4, 128


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------------------------------------ boundary -------

def test_flint_symbols_exported():
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b(mfl_[a-z0-9_]+)\s*\(", src)))
    assert sorted(mf.SYMBOLS) == names
    L = mf.lib()
    for n in names:
        assert hasattr(L, n)
    out = subprocess.run(["nm", "-D", "--defined-only", mk.LIB_PATH], capture_output=True, text=True).stdout
    assert set(names) <= set(re.findall(r" T (mfl_\w+)", out))


def test_flint_header_compiles_as_c():
    r = subprocess.run(["gcc", "-fsyntax-only", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), "-x", "c", HEADER],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_flint_errors_without_gpu():
    L = mf.lib()
    h = ctypes.c_void_p()
    mask = (ctypes.c_ubyte * 2)(1, 0)
    assert L.mfl_create(ctypes.byref(h), 2, 1500, mk.F32, mask, None) == mk.E_CTX
    assert L.mfl_create(ctypes.byref(h), 2, 4096, 5, mask, None) == mk.E_ARG
    assert L.mfl_create(ctypes.byref(h), 2, 4096, mk.F32, None, None) == mk.E_ARG
    assert L.mfl_attend(None, 0, 0, 1, None, None, None) == mk.E_ARG
    assert b"NULL" in L.mkv_last_error()


@pytest.mark.parametrize("pos", [0, 1, 513, 1023, 70000])
def test_flint_host_rope_table_matches_oracle(pos):
    assert np.array_equal(np.array(mf.rope_table(pos), np.float32), O.fl_rope_table(pos))


# ------------------------------------------------------------------------------------------------ RoPE -----------

@pytest.mark.parametrize("pos", [0, 3, 511, 40000])
def test_rope_table_is_the_f32_recurrence(pos):
    """theta_0 = pos, theta_{i+1} = theta_i * base^(-2/128) in f32; cos/sin within 1 ulp of float64 of that angle."""
    base = np.float32(10000.0)
    scale = np.float32(np.float64(base) ** (-2.0 / 128))
    t = O.fl_rope_table(pos, 10000.0)
    th = np.float32(pos)
    for i in range(64):
        c64, s64 = np.cos(np.float64(th)), np.sin(np.float64(th))
        assert abs(np.float64(t[i]) - c64) <= abs(np.spacing(np.float32(c64))) * 1.01 + 1e-45
        assert abs(np.float64(t[64 + i]) - s64) <= abs(np.spacing(np.float32(s64))) * 1.01 + 1e-45
        th = np.float32(th * scale)


def test_rope_rotates_pairs():
    x = rng(1).standard_normal((3, 5, D), dtype=np.float32)
    tabs = O.fl_rope_tables(0, 3)
    y = O.fl_rope(x, tabs)
    assert np.array_equal(y[0], x[0]), "position 0 is the identity"
    for t in range(3):
        c, s = tabs[t, :64].astype(np.float64), tabs[t, 64:].astype(np.float64)
        x0, x1 = x[t, :, :64].astype(np.float64), x[t, :, 64:].astype(np.float64)
        np.testing.assert_allclose(y[t, :, :64], x0 * c - x1 * s, atol=2e-6)  # pair (i, i + 64), first element
        np.testing.assert_allclose(y[t, :, 64:], x0 * s + x1 * c, atol=2e-6)
    n_in = x[..., :64] ** 2 + x[..., 64:] ** 2
    n_out = y[..., :64].astype(np.float64) ** 2 + y[..., 64:].astype(np.float64) ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5)


# ------------------------------------------------------------------------------------------------ writes ---------

@pytest.mark.parametrize("fmt", [0, 1])
def test_kv_write_ring_rows(fmt):
    ring = 1024
    kc, vc = O.fl_new_cache(ring, fmt), O.fl_new_cache(ring, fmt)
    k = rng(2).standard_normal((40, KVH, D), dtype=np.float32)
    v = rng(3).standard_normal((40, KVH, D), dtype=np.float32)
    O.fl_kv_write(fmt, kc, vc, 1000, k, v)  # positions 1000 .. 1039 wrap to rows 1000 .. 1023, 0 .. 15
    want_k = k if fmt == 1 else k.astype(np.float16).view(np.uint16)
    want_v = v if fmt == 1 else v.astype(np.float16).view(np.uint16)
    assert np.array_equal(kc[1000:], want_k[:24]) and np.array_equal(kc[:16], want_k[24:])
    assert np.array_equal(vc[1000:], want_v[:24]) and np.array_equal(vc[:16], want_v[24:])
    assert not kc[16:1000].any()


# ------------------------------------------------------------------------------------------------ attention ------

def fill_cache(fmt, rows, pos1, seed, scale=1.0):
    """Positions [0, pos1) written in blocks; returns the caches (reference layout)."""
    kc, vc = O.fl_new_cache(rows, fmt), O.fl_new_cache(rows, fmt)
    r = rng(seed)
    p = 0
    while p < pos1:
        n = min(512, pos1 - p)
        O.fl_kv_write(fmt, kc, vc, p, scale * r.standard_normal((n, KVH, D), dtype=np.float32),
                      r.standard_normal((n, KVH, D), dtype=np.float32))
        p += n
    return kc, vc


def as_f64(fmt, c):
    return (c.view(np.float16) if fmt == 0 else c).astype(np.float64)


def attn64(fmt, kc, vc, q, pos0, win, sinks):
    """float64 textbook: token t at pos0 + t sees positions [lo, pos] at rows pos % ring; the sink joins the maximum
    and the sum."""
    q = q.reshape(-1, H, D).astype(np.float64)
    K, Vv = as_f64(fmt, kc), as_f64(fmt, vc)
    ring = kc.shape[0]
    out = np.zeros(q.shape)
    for t in range(q.shape[0]):
        p = pos0 + t
        lo = O.fl_window_lo(p, win)
        rows = np.arange(lo, p + 1) % ring
        for h in range(H):
            g = h // 8
            s = K[rows, g] @ q[t, h] / np.sqrt(128.0)
            m = s.max() if sinks is None else max(s.max(), float(sinks[h]))
            e = np.exp(s - m)
            den = e.sum() + (0.0 if sinks is None else np.exp(float(sinks[h]) - m))
            out[t, h] = e @ Vv[rows, g] / den
    return out


@pytest.mark.parametrize("fmt,rows,pos,win", [(1, 4096, 3000, 0), (0, 4096, 700, 0), (1, 1024, 2500, 513),
                                              (0, 1024, 1100, 513), (1, 1024, 100, 513)])
def test_attn_fd_vs_float64(fmt, rows, pos, win):
    kc, vc = fill_cache(fmt, rows, pos + 1, seed=10 + pos)
    q = rng(11).standard_normal((H, D), dtype=np.float32)
    sinks = rng(12).standard_normal(H, dtype=np.float32)
    got = O.fl_attn_fd(fmt, kc, vc, q, pos, win, sinks)
    np.testing.assert_allclose(got, attn64(fmt, kc, vc, q, pos, win, sinks)[0], atol=2e-6, rtol=0)


@pytest.mark.parametrize("fmt,rows,pos0,n,win", [(1, 4096, 200, 70, 0), (0, 4096, 0, 9, 0), (1, 1024, 1900, 40, 513),
                                                 (0, 1024, 600, 33, 513)])
def test_attn_pf_vs_float64(fmt, rows, pos0, n, win):
    kc, vc = fill_cache(fmt, rows, pos0 + n, seed=20 + pos0)
    q = rng(21).standard_normal((n, H, D), dtype=np.float32)
    sinks = rng(22).standard_normal(H, dtype=np.float32)
    got = O.fl_attn_pf(fmt, kc, vc, q, pos0, win, sinks)
    np.testing.assert_allclose(got, attn64(fmt, kc, vc, q, pos0, win, sinks), atol=2e-6, rtol=0)


def test_sink_limits():
    """A very negative sink is no sink; a sink far above every score takes all the weight (output -> 0)."""
    kc, vc = fill_cache(1, 4096, 600, seed=30)
    q = rng(31).standard_normal((H, D), dtype=np.float32)
    plain = O.fl_attn_fd(1, kc, vc, q, 599, 0, None)
    np.testing.assert_allclose(O.fl_attn_fd(1, kc, vc, q, 599, 0, np.full(H, -1e30, np.float32)), plain, atol=1e-7)
    np.testing.assert_allclose(plain, attn64(1, kc, vc, q, 599, 0, None)[0], atol=2e-6)
    big = O.fl_attn_fd(1, kc, vc, q, 599, 0, np.full(H, 80.0, np.float32))
    assert np.abs(big).max() < 1e-25
    bigp = O.fl_attn_pf(1, kc, vc, q[None], 599, 0, np.full(H, 80.0, np.float32))
    assert np.abs(bigp).max() < 1e-25


def test_window_excludes_older_rows():
    """On a sliding ring, token at pos sees exactly [pos - 512, pos]: rewriting the ring rows of other positions
    leaves the output bit-identical, rewriting the oldest visible one changes it."""
    pos = 1500
    kc, vc = fill_cache(1, 1024, pos + 1, seed=40)
    q = rng(41).standard_normal((H, D), dtype=np.float32)
    sinks = rng(42).standard_normal(H, dtype=np.float32)
    a = O.fl_attn_fd(1, kc, vc, q, pos, 513, sinks)
    pa = O.fl_attn_pf(1, kc, vc, q[None], pos, 513, sinks)[0]
    k2, v2 = kc.copy(), vc.copy()
    hidden = [(p % 1024) for p in range(pos + 1 - 1024, pos - 512)]  # rows of positions before the window
    k2[hidden] = 1e3
    v2[hidden] = -7.0
    assert np.array_equal(O.fl_attn_fd(1, k2, v2, q, pos, 513, sinks), a)
    assert np.array_equal(O.fl_attn_pf(1, k2, v2, q[None], pos, 513, sinks)[0], pa)
    v3 = vc.copy()
    v3[(pos - 512) % 1024] += 5.0
    assert not np.array_equal(O.fl_attn_fd(1, kc, v3, q, pos, 513, sinks), a)


@pytest.mark.parametrize("fmt,rows,pos,win", [(1, 4096, 777, 0), (0, 1024, 3000, 513)])
def test_pf_of_one_token_is_fd(fmt, rows, pos, win):
    kc, vc = fill_cache(fmt, rows, pos + 1, seed=50)
    q = rng(51).standard_normal((H, D), dtype=np.float32)
    sinks = rng(52).standard_normal(H, dtype=np.float32)
    np.testing.assert_allclose(O.fl_attn_pf(fmt, kc, vc, q[None], pos, win, sinks)[0],
                               O.fl_attn_fd(fmt, kc, vc, q, pos, win, sinks), atol=1e-6)
