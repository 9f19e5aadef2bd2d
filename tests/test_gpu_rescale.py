"""The lazy reference max of the f16 kernels (attn_dmx / attn_fa_mx: the running max moves only when a tile's max
exceeds it by more than 8, dmx.rs:72-74) moving in the middle of a split: with N(0,1) keys scores never jump by 8,
so keys boosted 24x at a few positions force the rescale of O and of the row sums in decode_f16 and prefill_f16
(and the exact-max rescale of the f32 kernels). Checked against the oracle's restatement of the matching reference
kernel, at the task tolerance (f16 store) or within max-abs 1e-4 / relative 1e-5 (f32 store): with scores in the
hundreds, an exp argument shifted by 2^-22 of the score (the split products' rounding) already moves an output by a
few 1e-5, so the f32 store's usual 1e-5 max-abs bar is relaxed here, and only here, to 1e-4.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_attn_close, kv_inputs, q_inputs

pytestmark = pytest.mark.gpu

F16, F32 = 0, 1


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _store(torch, mk, fmt, npos, boost, seed):
    kn, v = kv_inputs(seed, npos)
    kn[boost] *= 24.0
    tab = O.rope_tables(0, npos)
    st = mk.KvStore(1, max(4096, (npos + 1023) // 1024 * 1024), fmt)
    for p in range(0, npos, 512):
        m = min(512, npos - p)
        st.append(0, p, _dev(torch, kn[p:p + m]), _dev(torch, v[p:p + m]), _dev(torch, tab[p:p + m]))
    kc, vc = O.new_cache(st.ctx, fmt), O.new_cache(st.ctx, fmt)
    O.append(fmt, kc, vc, 0, kn, v, tab)
    return st, kc, vc


@pytest.mark.parametrize("fmt", [F16, F32])
@pytest.mark.parametrize("n0,ntok", [(5000, 4), (5000, 1), (70000, 4)])
def test_decode_max_jump(torch_gpu, fmt, n0, ntok):
    import mechta_amd as mk
    torch = torch_gpu
    print(f"rescale decode fmt={fmt} n0={n0} ntok={ntok}", flush=True)
    npos = n0 + ntok - 1
    boost = [n0 // 3, n0 // 3 + 700, n0 - 2, npos - 1]
    st, kc, vc = _store(torch, mk, fmt, npos, boost, seed=91 + n0)
    with st:
        q = q_inputs(92, ntok)
        out = st.decode(0, _dev(torch, q), n0).cpu().numpy()
    if fmt == F32:
        assert_attn_close(out, O.attn_fd(F32, kc, vc, q, n0), atol=1e-4, rtol=1e-5, what="f32 decode, max jump")
    elif ntok == 1:
        assert_attn_close(out, O.attn_fd(F16, kc, vc, q, n0), what="f16 1-token decode, max jump")
    else:
        assert_attn_close(out, O.attn_dmx(kc, vc, q, n0), what="f16 decode, max jump")


@pytest.mark.parametrize("fmt", [F16, F32])
def test_prefill_max_jump(torch_gpu, fmt):
    import mechta_amd as mk
    torch = torch_gpu
    print(f"rescale prefill fmt={fmt}", flush=True)
    n0, T = 6000, 96
    npos = n0 - 1 + T
    boost = [1500, 3100, 5990, n0 + 40]
    st, kc, vc = _store(torch, mk, fmt, npos, boost, seed=93)
    with st:
        q = q_inputs(94, T)
        out = st.prefill(0, _dev(torch, q), n0).cpu().numpy()
    sel = np.array([0, 17, 39, 40, 41, 95], np.int32)
    if fmt == F32:
        assert_attn_close(out[sel], O.attn_fa_f32(kc, vc, q, n0, sel=sel), atol=1e-4, rtol=1e-5,
                          what="f32 prefill, max jump")
    else:
        assert_attn_close(out[sel], O.attn_fa_mx(kc, vc, q, n0, sel=sel), what="f16 prefill, max jump")


@pytest.mark.parametrize("fmt", [F16, F32])
@pytest.mark.parametrize("sliding", [False, True])
def test_flint_max_jump(torch_gpu, fmt, sliding):
    """The Flint kernels (exact running max, sinks) with keys boosted 24x: one-token decode and a 64-token block."""
    from mechta_amd import flint as mf
    torch = torch_gpu
    print(f"rescale flint fmt={fmt} sliding={sliding}", flush=True)
    H, KVH, D = 32, 4, 128
    npos = 2600
    r = np.random.default_rng(95)
    k = r.standard_normal((npos, KVH, D), dtype=np.float32)
    v = r.standard_normal((npos, KVH, D), dtype=np.float32)
    for b in (700, 2200, 2400, npos - 1):
        k[b] *= 24.0
    sinks = r.standard_normal(H, dtype=np.float32)
    win = 513 if sliding else 0
    with mf.FlintStore(1, 4096, fmt, sliding=[sliding]) as st:
        rows = st.rows(0)
        kc, vc = O.fl_new_cache(rows, fmt), O.fl_new_cache(rows, fmt)
        for p in range(0, npos - 64, 512):
            m = min(512, npos - 64 - p)
            st.append(0, p, _dev(torch, k[p:p + m]), _dev(torch, v[p:p + m]))
            O.fl_kv_write(fmt, kc, vc, p, k[p:p + m], v[p:p + m])
        p0 = npos - 64
        st.append(0, p0, _dev(torch, k[p0:]), _dev(torch, v[p0:]))
        O.fl_kv_write(fmt, kc, vc, p0, k[p0:], v[p0:])
        q = r.standard_normal((64, H, D), dtype=np.float32)
        blk = st.attend(0, p0, _dev(torch, q), _dev(torch, sinks)).cpu().numpy()
        one = st.attend(0, npos - 1, _dev(torch, q[-1:]), _dev(torch, sinks)).cpu().numpy()
    tol = dict(atol=1e-4, rtol=1e-5)
    assert_attn_close(blk, O.fl_attn_pf(fmt, kc, vc, q, p0, win, sinks), what="flint block, max jump", **tol)
    assert_attn_close(one[0], O.fl_attn_fd(fmt, kc, vc, q[-1], npos - 1, win, sinks), what="flint one token, max jump",
                      **tol)
