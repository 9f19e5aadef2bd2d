"""Seeded random sweep of the KV-cache path through the C ABI against the CPU oracle: append lengths, decode token
counts and windows, prefill blocks, both store formats, at sizes the oracle finishes quickly. Bars as in
test_gpu_kvpath.py: appended rows bit-exact; f16 attention within max-abs 2e-3 / relative 1e-3 of the oracle's
restatement of the matching reference kernel (attn_dmx, attn_fd with a window, attn_fa_mx), f32 within 1e-5.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_attn_close, kv_inputs, prefill_reference, q_inputs

pytestmark = pytest.mark.gpu

F16, F32 = 0, 1


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _rows(st, which, p1):
    t = st.read_rows(0, which, 0, p1).cpu().numpy()
    return t.view(np.uint16) if t.dtype == np.int16 else t


def _cases(seed, count):
    r = np.random.default_rng(seed)
    out = []
    for i in range(count):
        fmt = int(r.integers(0, 2))
        n0 = int(r.integers(1, 12000))
        ntok = int(r.integers(1, 5))
        start = 0 if r.random() < 0.6 else int(r.integers(0, n0))
        out.append((i, fmt, n0, ntok, start))
    return out


@pytest.mark.parametrize("i,fmt,n0,ntok,start", _cases(2027, 24))
def test_sweep_append_decode(torch_gpu, i, fmt, n0, ntok, start):
    import mechta_amd as mk
    torch = torch_gpu
    print(f"sweep decode #{i} fmt={fmt} n0={n0} ntok={ntok} start={start}", flush=True)
    npos = n0 + ntok - 1
    ctx = max(4096, (npos + 1023) // 1024 * 1024)
    kn, v = kv_inputs(5000 + i, npos)
    tab = O.rope_tables(0, npos)
    q = q_inputs(6000 + i, ntok)
    r = np.random.default_rng(7000 + i)
    with mk.KvStore(1, ctx, fmt) as st:
        p = 0
        while p < n0 - 1:  # ragged appends of the prefix
            m = min(int(r.integers(1, 513)), n0 - 1 - p)
            st.append(0, p, _dev(torch, kn[p:p + m]), _dev(torch, v[p:p + m]), _dev(torch, tab[p:p + m]))
            p += m
        out = st.append_decode(0, n0, _dev(torch, kn[n0 - 1:]), _dev(torch, v[n0 - 1:]), _dev(torch, tab[n0 - 1:]),
                               _dev(torch, q), start=start).cpu().numpy()
        kg, vg = _rows(st, mk.K, npos), _rows(st, mk.V, npos)
    kc, vc = O.new_cache(ctx, fmt), O.new_cache(ctx, fmt)
    O.append(fmt, kc, vc, 0, kn, v, tab)
    assert np.array_equal(kg, kc[:npos]) and np.array_equal(vg, vc[:npos]), "appended rows differ"
    if fmt == F32:
        assert_attn_close(out, O.attn_fd(F32, kc, vc, q, n0, start=start), atol=1e-5, rtol=1e-5, what="f32")
    elif start == 0:
        assert_attn_close(out, O.attn_dmx(kc, vc, q, n0), what="f16 vs attn_dmx")
    else:
        assert_attn_close(out, O.attn_fd(F16, kc, vc, q, n0, start=start), what="f16 window vs attn_fd")


def _pf_cases(seed, count):
    r = np.random.default_rng(seed)
    out = []
    for i in range(count):
        fmt = int(r.integers(0, 2))
        T = int(r.integers(1, 513))
        n0 = int(r.integers(1, 6000))
        start = 0 if r.random() < 0.7 else int(r.integers(0, n0))
        out.append((i, fmt, n0, T, start))
    return out


@pytest.mark.parametrize("i,fmt,n0,T,start", _pf_cases(2028, 12))
def test_sweep_prefill(torch_gpu, i, fmt, n0, T, start):
    import mechta_amd as mk
    torch = torch_gpu
    print(f"sweep prefill #{i} fmt={fmt} n0={n0} T={T} start={start}", flush=True)
    npos = n0 - 1 + T
    ctx = max(4096, (npos + 1023) // 1024 * 1024)
    kn, v = kv_inputs(8000 + i, npos)
    tab = O.rope_tables(0, npos)
    q = q_inputs(9000 + i, T)
    sel = np.unique(np.r_[0, T - 1, np.random.default_rng(i).integers(0, T, 6)]).astype(np.int32)
    with mk.KvStore(1, ctx, fmt) as st:
        for p in range(0, npos, 512):
            m = min(512, npos - p)
            st.append(0, p, _dev(torch, kn[p:p + m]), _dev(torch, v[p:p + m]), _dev(torch, tab[p:p + m]))
        out = st.prefill(0, _dev(torch, q), n0, start=start).cpu().numpy()
    kc, vc = O.new_cache(ctx, fmt), O.new_cache(ctx, fmt)
    O.append(fmt, kc, vc, 0, kn, v, tab)
    ref, atol, rtol = prefill_reference(fmt, kc, vc, q, n0, start=start, sel=sel)
    assert_attn_close(out[sel], ref, atol=atol, rtol=rtol, what=f"prefill fmt {fmt} T {T}")
