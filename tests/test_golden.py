"""Golden vectors of the KV-cache path (tests/golden/fixtures.npz, written by tests/golden/gen_fixtures.py).

CPU: the input generator is pinned by the published SplitMix64 vectors and by its distribution, and the oracle still
reproduces every stored output. GPU: the HIP path, through the C ABI, matches the stored outputs: appended rows and
row hashes bit-exact, attention within max-abs 2e-3 / relative 1e-3 (Flint: 1e-5 / 1e-5, f32-class arithmetic).
"""
import hashlib
import os

import numpy as np
import pytest

from tests.golden import gen_fixtures as G
from tests.helpers import assert_attn_close

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="module")
def xs():
    return G.inputs()


def test_splitmix64_known_answers():
    """SplitMix64 with state 1234567 (state += 0x9E3779B97F4A7C15, output = finalizer(state)): the published first
    five outputs (Vigna's reference implementation)."""
    s = np.array([1234567], np.uint64)
    g = np.uint64(0x9E3779B97F4A7C15)
    with np.errstate(over="ignore"):
        got = [int(G._mix(s + g * np.uint64(k))[0]) for k in range(1, 6)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
                   16408922859458223821]


def test_normals_distribution_and_pins(fx):
    from scipy import stats
    x = G.normals(7, (1 << 18,)).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.var() - 1.0) < 0.01
    assert stats.kstest(x, "norm").pvalue > 1e-3
    assert not np.array_equal(G.normals(7, (64,)), G.normals(8, (64,)))
    assert np.array_equal(G.generator_pins(), fx["gen_pins"])


def test_oracle_reproduces_fixtures(fx, xs):
    e = G.expected(xs)
    for k in ("append4_k", "append4_v", "append4_sha_k", "append4_sha_v", "rows_f32_sha"):
        assert np.array_equal(e[k], fx[k]), k
    for k in ("decode4", "decode1_gate", "prefill64", "flint_full", "flint_slide"):
        np.testing.assert_allclose(e[k], fx[k], rtol=1e-6, atol=1e-7, err_msg=k)


# ------------------------------------------------------------------------------------------------- GPU ------

def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _sha(t):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(t).tobytes()).digest(), np.uint8)


def _fill(torch, mk, st, layer, kn, v, p0=0):
    from oracle import oracle as O  # RoPE table rows (host f32 table, rope_table): the reference's caller input
    n = kn.shape[0]
    tab = O.rope_tables(p0, n)
    for a in range(0, n, mk.PREFILL_MAX):
        b = min(a + mk.PREFILL_MAX, n)
        st.append(layer, p0 + a, _dev(torch, kn[a:b]), _dev(torch, v[a:b]), _dev(torch, tab[a:b]))


def _rows(st, layer, which, p1):
    t = st.read_rows(layer, which, 0, p1).cpu().numpy()
    return t.view(np.uint16) if t.dtype == np.int16 else t


@pytest.mark.gpu
def test_gpu_append_decode4(torch_gpu, fx, xs):
    import mechta_amd as mk
    from oracle import oracle as O
    torch = torch_gpu
    print("golden append4 + decode4", flush=True)
    with mk.KvStore(1, 4096, mk.F16) as st:
        _fill(torch, mk, st, 0, xs["kn300"], xs["v300"])
        out = st.append_decode(0, 301, _dev(torch, xs["kn4"]), _dev(torch, xs["v4"]),
                               _dev(torch, O.rope_tables(300, 4)), _dev(torch, xs["q4"])).cpu().numpy()
        k, v = _rows(st, 0, mk.K, 304), _rows(st, 0, mk.V, 304)
    assert np.array_equal(k[300:], fx["append4_k"]) and np.array_equal(v[300:], fx["append4_v"])
    assert np.array_equal(_sha(k), fx["append4_sha_k"]) and np.array_equal(_sha(v), fx["append4_sha_v"])
    assert_attn_close(out, fx["decode4"], what="golden decode4")


@pytest.mark.gpu
def test_gpu_decode1_gate(torch_gpu, fx, xs):
    import mechta_amd as mk
    from oracle import oracle as O
    torch = torch_gpu
    print("golden decode1 + gate", flush=True)
    with mk.KvStore(1, 4096, mk.F16) as st:
        _fill(torch, mk, st, 0, xs["kn1k"], xs["v1k"])
        out = st.append_decode(0, 1001, _dev(torch, xs["kn1"]), _dev(torch, xs["v1"]),
                               _dev(torch, O.rope_tables(1000, 1)), _dev(torch, xs["q1"]),
                               gate_src=_dev(torch, xs["gate1"])).cpu().numpy()
    assert_attn_close(out, fx["decode1_gate"], what="golden decode1 gate")


@pytest.mark.gpu
def test_gpu_prefill64(torch_gpu, fx, xs):
    import mechta_amd as mk
    torch = torch_gpu
    print("golden prefill64", flush=True)
    with mk.KvStore(1, 4096, mk.F16) as st:
        _fill(torch, mk, st, 0, xs["kn2k"], xs["v2k"])
        _fill(torch, mk, st, 0, xs["kn64"], xs["v64"], p0=2000)
        out = st.prefill(0, _dev(torch, xs["q64"]), 2001, scale=1.0).cpu().numpy()
    assert_attn_close(out[fx["pf_sel"]], fx["prefill64"], what="golden prefill64")


@pytest.mark.gpu
def test_gpu_rows_f32(torch_gpu, fx, xs):
    import mechta_amd as mk
    torch = torch_gpu
    print("golden rows f32", flush=True)
    with mk.KvStore(3, 4096, mk.F32) as st:
        for layer, (kn, v) in enumerate(xs["f32rows"]):
            _fill(torch, mk, st, layer, kn, v)
        for layer in range(3):
            assert np.array_equal(_sha(_rows(st, layer, mk.K, 256)), fx["rows_f32_sha"][layer, 0])
            assert np.array_equal(_sha(_rows(st, layer, mk.V, 256)), fx["rows_f32_sha"][layer, 1])


@pytest.mark.gpu
def test_gpu_flint(torch_gpu, fx, xs):
    from mechta_amd import flint as mf
    torch = torch_gpu
    print("golden flint full + sliding", flush=True)
    sinks = _dev(torch, xs["fl_sinks"])
    with mf.FlintStore(1, 4096, mf.F32, sliding=[False]) as st:
        st.append(0, 0, _dev(torch, xs["fl_full_k"]), _dev(torch, xs["fl_full_v"]))
        out = st.attend(0, 299, _dev(torch, xs["fl_full_q"][None]), sinks).cpu().numpy()
    assert_attn_close(out[0], fx["flint_full"], atol=1e-5, rtol=1e-5, what="golden flint full")
    with mf.FlintStore(1, 4096, mf.F16, sliding=[True]) as st:
        for a in range(0, 1500, 512):
            b = min(a + 512, 1500)
            st.append(0, a, _dev(torch, xs["fl_slide_k"][a:b]), _dev(torch, xs["fl_slide_v"][a:b]))
        out = st.attend(0, 1499, _dev(torch, xs["fl_slide_q"][None]), sinks).cpu().numpy()
    assert_attn_close(out[0], fx["flint_slide"], atol=1e-5, rtol=1e-5, what="golden flint sliding")
