"""GPU parity tests of the KV-cache path through the C ABI (libmechta_kv.so), against the CPU oracle.

Bars: append bit-exact to the oracle (f32 -> f16 round to nearest even, RoPE without FMA); attention within
max-abs 2e-3 and relative 1e-3 of the oracle restatement of the reference kernel for the same path (attn_fd for one
f32-semantics token, attn_dmx for the f16 4-token verify, attn_fa_mx for the prefill); snapshot bit-identical.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import (SMALL_PREFILL_MAX, assert_attn_close, err_stats, exact_attention, gate_inputs, kv_inputs,
                           prefill_reference, q_inputs, read_root_py, write_root_py)

pytestmark = pytest.mark.gpu

F16, F32 = 0, 1


@pytest.fixture(scope="module")
def mk(torch_gpu):
    import mechta_amd
    mechta_amd.lib()
    return mechta_amd


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def fill(torch, store, layer, fmt, n_pos, seed, chunks=(512,), oracle_caches=None):
    """Appends n_pos seeded tokens to `layer` through the GPU path (in appends of the given sizes, cycled) and, if
    oracle_caches is given, through the oracle too. Returns the inputs."""
    kn, v = kv_inputs(seed, n_pos)
    tab = O.rope_tables(0, n_pos)
    pos, i = 0, 0
    while pos < n_pos:
        m = min(chunks[i % len(chunks)], n_pos - pos)
        store.append(layer, pos, dev(torch, kn[pos:pos + m]), dev(torch, v[pos:pos + m]), dev(torch, tab[pos:pos + m]))
        pos += m
        i += 1
    if oracle_caches is not None:
        kc, vc = oracle_caches
        O.append(fmt, kc, vc, 0, kn, v, tab)
    return kn, v, tab


def rows_np(store, layer, which, p0, p1):
    t = store.read_rows(layer, which, p0, p1).cpu().numpy()
    return t.view(np.uint16) if t.dtype == np.int16 else t


def caches_np(store, layer, p1):
    return rows_np(store, layer, 0, 0, p1), rows_np(store, layer, 1, 0, p1)


# ------------------------------------------------------------------------------------------------ append ---------

@pytest.mark.parametrize("fmt", [F16, F32])
def test_append_bit_exact(torch_gpu, mk, fmt):
    torch = torch_gpu
    print(f"append fmt={fmt}", flush=True)
    ctx, n_pos = 4096, 1000
    kc, vc = O.new_cache(ctx, fmt), O.new_cache(ctx, fmt)
    with mk.KvStore(2, ctx, fmt) as st:
        # ragged appends: 1, 3, 4, 64, 7, 512 ... cross every block / group boundary of the store layout
        fill(torch, st, 1, fmt, n_pos, seed=11, chunks=(1, 3, 4, 64, 7, 512, 2), oracle_caches=(kc, vc))
        st.sync()
        gk, gv = caches_np(st, 1, n_pos)
        assert np.array_equal(gk, kc[:n_pos]), "K differs"
        assert np.array_equal(gv, vc[:n_pos]), "V differs"
        # layer 0 untouched
        assert st.length(0) == 0 and st.length(1) == n_pos
        assert not np.any(rows_np(st, 0, 0, 0, 64))


def test_append_f16_special_values(torch_gpu, mk):
    """Values at the f16 boundaries: overflow to inf, the largest finite, subnormals, ties, signed zero."""
    torch = torch_gpu
    specials = np.array([65504.0, 65519.99, 65520.0, 1e6, -1e6, 6.1035156e-05, 6.1e-05, 5.96e-08, 2.98e-08,
                         2.99e-08, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, -0.0, 0.0, 1e-30, 3.14159265, -2.7182817],
                        np.float32)
    r = np.random.default_rng(5)
    ntok = 8
    kn = r.choice(specials, size=(ntok, 2, 256)).astype(np.float32)
    v = r.choice(specials, size=(ntok, 512)).astype(np.float32)
    tab = O.rope_tables(0, ntok)
    kc, vc = O.new_cache(4096, F16), O.new_cache(4096, F16)
    O.append(F16, kc, vc, 0, kn, v, tab)
    with mk.KvStore(1, 4096, F16) as st:
        st.append(0, 0, dev(torch, kn), dev(torch, v), dev(torch, tab))
        gk, gv = caches_np(st, 0, ntok)
    assert np.array_equal(gk, kc[:ntok]) and np.array_equal(gv, vc[:ntok])


def test_append_rollback(torch_gpu, mk):
    """Rejected drafts: append 4 at pos, keep 2 (set_len), append 4 at pos + 2: same cache as a clean sequence."""
    torch = torch_gpu
    ctx, n0 = 4096, 300
    kn, v = kv_inputs(21, n0 + 8)
    knb, vb = kv_inputs(22, 4)  # the rejected drafts' rows
    tab = O.rope_tables(0, n0 + 8)
    with mk.KvStore(1, ctx, F16) as a, mk.KvStore(1, ctx, F16) as b:
        # a: the step at n0 wrote 4 rows, the sure token and 3 drafts; the first draft is accepted, the last two
        # (rows n0 + 2, n0 + 3) are rejected
        a.append(0, 0, dev(torch, kn[:n0 + 2]), dev(torch, v[:n0 + 2]), dev(torch, tab[:n0 + 2]))
        a.append(0, n0 + 2, dev(torch, knb[:2]), dev(torch, vb[:2]), dev(torch, tab[n0 + 2:n0 + 4]))
        b.append(0, 0, dev(torch, kn[:n0 + 2]), dev(torch, v[:n0 + 2]), dev(torch, tab[:n0 + 2]))
        a.set_len(n0 + 2)
        assert a.length() == n0 + 2
        a.append(0, n0 + 2, dev(torch, kn[n0 + 2:n0 + 6]), dev(torch, v[n0 + 2:n0 + 6]), dev(torch, tab[n0 + 2:n0 + 6]))
        b.append(0, n0 + 2, dev(torch, kn[n0 + 2:n0 + 6]), dev(torch, v[n0 + 2:n0 + 6]), dev(torch, tab[n0 + 2:n0 + 6]))
        ka, va = caches_np(a, 0, n0 + 6)
        kb, vb2 = caches_np(b, 0, n0 + 6)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb2)
        q = dev(torch, q_inputs(23, 4))
        oa = a.decode(0, q, n0 + 3).cpu().numpy()
        ob = b.decode(0, q, n0 + 3).cpu().numpy()
        assert np.array_equal(oa, ob)


def test_errors(torch_gpu, mk):
    torch = torch_gpu
    with pytest.raises(mk.MkvError) as e:
        mk.KvStore(1, 5000, F16)
    assert e.value.code == mk.E_CTX
    with mk.KvStore(2, 4096, F16) as st:
        kn, v = kv_inputs(1, 4)
        tab = O.rope_tables(0, 4)
        args = (dev(torch, kn), dev(torch, v), dev(torch, tab))
        with pytest.raises(mk.MkvError) as e:
            st.append(0, 10, *args)  # hole
        assert e.value.code == mk.E_POS
        with pytest.raises(mk.MkvError) as e:
            st.append(2, 0, *args)
        assert e.value.code == mk.E_LAYER
        st.append(0, 0, *args)
        q = dev(torch, q_inputs(2, 4))
        with pytest.raises(mk.MkvError) as e:
            st.decode(0, q, 2)  # reads up to 5 > 4
        assert e.value.code == mk.E_POS
        with pytest.raises(mk.MkvError) as e:
            st.set_len(5)
        assert e.value.code == mk.E_POS
        with pytest.raises(mk.MkvError) as e:
            st.restore(4, torch.empty(3, dtype=torch.uint8, pin_memory=True))
        assert e.value.code == mk.E_SIZE
        with pytest.raises(ValueError):  # pageable host memory: refused before any copy
            st.restore(4, torch.empty(st.snapshot_bytes(4), dtype=torch.uint8))


# ------------------------------------------------------------------------------------------------ decode ---------

DECODE_CASES = [  # (ctx, n0 positions already in the cache, ntok, start)
    (4096, 1, 1, 0), (4096, 31, 4, 0), (4096, 300, 4, 0), (4096, 1000, 1, 0), (4096, 4092, 4, 0),
    (8192, 4096, 1, 0), (8192, 5000, 4, 0), (8192, 2047, 2, 0), (8192, 3000, 3, 1), (8192, 3000, 4, 700),
    (20480, 20000, 4, 0), (20480, 17000, 1, 0),
    # 64-key stages dealt to 108 work-groups per kv head: 1150 stages leave a partial round of 70 > 108 / 2 (whole
    # stages), 1092 a round of 12 and 1026 a round of 54 = 108 / 2 (split into half stages)
    (74752, 73590, 4, 0), (70656, 69885, 4, 0), (66560, 65660, 4, 0), (66560, 65600, 1, 3000),
]


@pytest.mark.parametrize("ctx,n0,ntok,start", DECODE_CASES)
def test_decode_f16(torch_gpu, mk, ctx, n0, ntok, start):
    torch = torch_gpu
    print(f"decode f16 ctx={ctx} n0={n0} ntok={ntok} start={start}", flush=True)
    with mk.KvStore(1, ctx, F16) as st:
        fill(torch, st, 0, F16, n0 + ntok - 1 if n0 + ntok - 1 > 0 else 1, seed=100 + n0)
        q = q_inputs(200 + n0, ntok)
        out = st.decode(0, dev(torch, q), n0, start=start).cpu().numpy()
        kc, vc = caches_np(st, 0, n0 + ntok - 1)
    ref = O.attn_dmx(kc, vc, q, n0) if start == 0 else O.attn_fd(F16, kc, vc, q, n0, start=start)
    assert_attn_close(out, ref, what="vs oracle")
    ex = exact_attention(kc, vc, q, n0, start=start)
    assert_attn_close(out, ex, what="vs f64")
    if ntok == 1:
        assert_attn_close(out, O.attn_fd(F16, kc, vc, q, n0, start=start), what="vs attn_fd")


def test_decode_split_count_sequence(torch_gpu, mk):
    """A sequence of decodes on one store whose split counts repeat and alternate (108, 79, 108, 79 with one token,
    47, 108, 79, 108 with one token, 108): every output against the oracle (the workspace is shared by all of them)."""
    torch = torch_gpu
    with mk.KvStore(1, 12288, F16) as st:
        fill(torch, st, 0, F16, 10000, seed=77)
        kc, vc = caches_np(st, 0, 10000)
        for i, (n0, ntok) in enumerate([(9000, 4), (5000, 4), (9000, 4), (5000, 1), (3000, 4), (9000, 4), (5000, 4),
                                        (9000, 1), (9000, 4)]):
            print(f"split count sequence step {i}: n0={n0} ntok={ntok}", flush=True)
            q = q_inputs(500 + i, ntok)
            out = st.decode(0, dev(torch, q), n0).cpu().numpy()
            ref = O.attn_dmx(kc, vc, q, n0) if ntok > 1 else O.attn_fd(F16, kc, vc, q, n0)
            assert np.isfinite(out).all(), f"step {i}: non-finite output"
            assert_attn_close(out, ref, what=f"step {i}")


@pytest.mark.parametrize("ctx,n0,ntok,start", [(4096, 300, 4, 0), (4096, 1000, 1, 0), (8192, 5000, 4, 17),
                                               (4096, 2, 1, 0), (4096, 129, 2, 0), (20480, 19000, 3, 0),
                                               (20480, 19001, 4, 12345), (8192, 40, 4, 33),
                                               (4096, 4093, 4, 0), (4096, 4096, 1, 0)])  # up to the context's end
def test_decode_f32(torch_gpu, mk, ctx, n0, ntok, start):
    torch = torch_gpu
    print(f"decode f32 ctx={ctx} n0={n0} ntok={ntok}", flush=True)
    with mk.KvStore(1, ctx, F32) as st:
        fill(torch, st, 0, F32, n0 + ntok - 1, seed=300 + n0)
        q = q_inputs(400 + n0, ntok)
        out = st.decode(0, dev(torch, q), n0, start=start).cpu().numpy()
        kc, vc = caches_np(st, 0, n0 + ntok - 1)
    ref = O.attn_fd(F32, kc, vc, q, n0, start=start)
    assert_attn_close(out, ref, atol=1e-5, rtol=1e-5, what="f32 vs attn_fd")


def test_decode_gate(torch_gpu, mk):
    torch = torch_gpu
    n0, ntok = 777, 4
    with mk.KvStore(1, 4096, F16) as st:
        fill(torch, st, 0, F16, n0 + ntok - 1, seed=5)
        q = q_inputs(6, ntok)
        qf = gate_inputs(7, ntok)
        out = st.decode(0, dev(torch, q), n0, gate_src=dev(torch, qf)).cpu().numpy()
        kc, vc = caches_np(st, 0, n0 + ntok - 1)
    ref = O.gate(O.attn_dmx(kc, vc, q, n0), qf).reshape(out.shape)
    assert_attn_close(out, ref, what="gated")


@pytest.mark.parametrize("fmt,ctx,n0,ntok,start", [(F16, 4096, 777, 4, 0), (F16, 66560, 65537, 4, 0),
                                                   (F16, 4096, 3000, 2, 0), (F16, 4096, 2000, 1, 500),
                                                   (F32, 4096, 1500, 4, 0)])
def test_gate16_output(torch_gpu, mk, fmt, ctx, n0, ntok, start):
    """The gated attention as f16 (mkv_append_decode_g16 / mkv_decode_g16, the reference's attn_gate16 of the 4-token
    verify, quad.rs:125, and of the f16 2-token step, engine.rs:1103): bit for bit the round-to-nearest-even f16 of
    the f32 entry points' gated output, and within the attention bar of orc_gate16 over the oracle's attention."""
    torch = torch_gpu
    print(f"gate16 fmt={fmt} ctx={ctx} n0={n0} ntok={ntok} start={start}", flush=True)
    kn, v = kv_inputs(41, ntok)
    tab = O.rope_tables(n0 - 1, ntok)
    q, qf = q_inputs(42, ntok), gate_inputs(43, ntok)
    with mk.KvStore(1, ctx, fmt) as a, mk.KvStore(1, ctx, fmt) as b:
        fill(torch, a, 0, fmt, n0 - 1, seed=44)
        fill(torch, b, 0, fmt, n0 - 1, seed=44)
        args = (0, n0, dev(torch, kn), dev(torch, v), dev(torch, tab), dev(torch, q))
        h = a.append_decode(*args, start=start, gate_src=dev(torch, qf), f16_out=True).cpu().numpy()
        f = b.append_decode(*args, start=start, gate_src=dev(torch, qf)).cpu().numpy()
        assert h.dtype == np.float16
        assert np.array_equal(h.view(np.uint16), f.astype(np.float16).view(np.uint16))
        h2 = a.decode(0, dev(torch, q), n0, start=start, gate_src=dev(torch, qf), f16_out=True).cpu().numpy()
        assert np.array_equal(h2.view(np.uint16), h.view(np.uint16))
        with pytest.raises(mk.MkvError):
            a.decode(0, dev(torch, q), n0, start=start, f16_out=True)  # the f16 output is the gated one
        kc, vc = caches_np(a, 0, n0 + ntok - 1) if ctx <= 8192 else (None, None)
    if kc is not None:
        if fmt == F32 or ntok == 1 or start > 0:
            att = O.attn_fd(fmt, kc, vc, q, n0, start=start)
        else:
            att = O.attn_dmx(kc, vc, q, n0)
        ref = O.gate16(att, qf).view(np.float16).astype(np.float32).reshape(h.shape)
        assert_attn_close(h.astype(np.float32), ref, atol=2e-3, rtol=2e-3, what="gate16")


@pytest.mark.parametrize("fmt", [F16, F32])
@pytest.mark.parametrize("ctx,n0", [(4096, 1234), (4096, 1279), (4096, 1282), (4096, 66), (20480, 19199),
                                    (66560, 65536 + 63)])
def test_append_decode_fused_entry(torch_gpu, mk, ctx, n0, fmt):
    """The fused entry equals append + decode bit for bit, also when the new rows straddle two 64-key stages (f16) or
    32-key tiles (f32) held by different work-groups, or sit in a work-group's first stages."""
    torch = torch_gpu
    print(f"fused append+decode fmt={fmt} ctx={ctx} n0={n0}", flush=True)
    kn, v = kv_inputs(31, 4)
    tab = O.rope_tables(n0 - 1, 4)
    q = q_inputs(32, 4)
    with mk.KvStore(1, ctx, fmt) as a, mk.KvStore(1, ctx, fmt) as b:
        fill(torch, a, 0, fmt, n0 - 1, seed=33)
        fill(torch, b, 0, fmt, n0 - 1, seed=33)
        oa = a.append_decode(0, n0, dev(torch, kn), dev(torch, v), dev(torch, tab), dev(torch, q)).cpu().numpy()
        b.append(0, n0 - 1, dev(torch, kn), dev(torch, v), dev(torch, tab))
        ob = b.decode(0, dev(torch, q), n0).cpu().numpy()
        ka, va = caches_np(a, 0, n0 + 3)
        kb, vb = caches_np(b, 0, n0 + 3)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb), "fused append wrote other rows"
    assert np.array_equal(oa, ob)
    if fmt == F16:
        assert_attn_close(oa, O.attn_dmx(ka, va, q, n0), what="fused vs oracle")
    else:
        assert_attn_close(oa, O.attn_fd(F32, ka, va, q, n0), atol=1e-5, rtol=1e-5, what="fused f32 vs oracle")


# ------------------------------------------------------------------------------------------------ prefill --------

@pytest.mark.parametrize("n0,T,start", [(2000, 64, 0), (100, 512, 0), (3000, 37, 0), (1, 16, 0), (2500, 96, 300),
                                        (3000, 63, 0), (1, 1, 0), (2001, 8, 0), (1000, 32, 0), (3500, 5, 0),
                                        (3000, 29, 1234), (60, 2, 0), (2000, 64, 700),
                                        (3585, 512, 0), (4090, 7, 0), (4033, 64, 1000)])  # the last three end at ctx
def test_prefill_f16(torch_gpu, mk, n0, T, start):
    """Blocks of 64 tokens or more against attn_fa_mx (f16 Q), smaller blocks against attn_fd4 (f32 Q) at 1e-5."""
    torch = torch_gpu
    print(f"prefill f16 n0={n0} T={T} start={start}", flush=True)
    with mk.KvStore(1, 4096, F16) as st:
        fill(torch, st, 0, F16, n0 + T - 1, seed=500 + T)
        q = q_inputs(600 + T, T)
        out = st.prefill(0, dev(torch, q), n0, start=start).cpu().numpy()
        kc, vc = caches_np(st, 0, n0 + T - 1)
    ref, atol, rtol = prefill_reference(F16, kc, vc, q, n0, start=start)
    assert_attn_close(out, ref, atol=atol, rtol=rtol, what=f"prefill T {T} vs its reference kernel")
    if T <= SMALL_PREFILL_MAX:  # f32 Q really used: the f16-Q prefill of the same block is further from float64
        ex = exact_attention(kc, vc, q, n0, start=start)
        assert err_stats(out, ex)[0] <= 1e-5


@pytest.mark.parametrize("n0,T,start", [(1500, 70, 0), (100, 512, 0), (2500, 96, 300), (1, 16, 0), (3000, 5, 0),
                                        (40, 3, 0), (3500, 512, 2900), (1500, 70, 400),
                                        (3585, 512, 0), (4092, 5, 0)])  # the last two end at ctx
def test_prefill_f32(torch_gpu, mk, n0, T, start):
    torch = torch_gpu
    print(f"prefill f32 n0={n0} T={T} start={start}", flush=True)
    with mk.KvStore(1, 4096, F32) as st:
        fill(torch, st, 0, F32, n0 + T - 1, seed=700 + T)
        q = q_inputs(701 + T, T)
        out = st.prefill(0, dev(torch, q), n0, start=start).cpu().numpy()
        kc, vc = caches_np(st, 0, n0 + T - 1)
    ref = O.attn_fa_f32(kc, vc, q, n0, start=start)
    assert_attn_close(out, ref, atol=1e-5, rtol=1e-5, what="prefill f32")


@pytest.mark.parametrize("fmt", [F16, F32])
def test_stale_nan_rows_past_the_length(torch_gpu, mk, fmt):
    """Rows past the written length (rejected drafts, never-written memory) may hold anything, NaN included: decode
    and prefill read whole blocks and must keep those rows out of the results."""
    torch = torch_gpu
    n0, ntok = 1000, 4
    with mk.KvStore(1, 4096, fmt) as st:
        fill(torch, st, 0, fmt, n0 + 100, seed=41)
        nan = torch.full((102 - ntok, 2, 256), float("nan"), device="cuda")
        if fmt == F16:
            nan = nan.half().view(torch.int16)
        for which in (0, 1):
            st.write_rows(0, which, n0 + ntok - 1, n0 + 101, nan)
        st.set_len(n0 + ntok - 1)
        q = q_inputs(42, ntok)
        out = st.decode(0, dev(torch, q), n0).cpu().numpy()
        outs = []
        for T in (40, 80):  # a small block (f32-class) and a matrix-unit block
            qp = q_inputs(43 + T, T)
            outs.append((qp, T, st.prefill(0, dev(torch, qp), n0 + ntok - T).cpu().numpy()))
        kc, vc = caches_np(st, 0, n0 + ntok - 1)
    if fmt == F16:
        assert_attn_close(out, O.attn_dmx(kc, vc, q, n0), what="decode next to NaN rows")
    else:
        assert_attn_close(out, O.attn_fd(F32, kc, vc, q, n0), atol=1e-5, rtol=1e-5, what="decode next to NaN rows")
    for qp, T, outp in outs:
        ref, atol, rtol = prefill_reference(fmt, kc, vc, qp, n0 + ntok - T)
        assert_attn_close(outp, ref, atol=atol, rtol=rtol, what=f"prefill of {T} next to NaN rows")


# ------------------------------------------------------------------------------------------------ snapshot -------

def test_snapshot_refuses_unpinned_host_memory(torch_gpu, mk):
    """The C ABI itself refuses a pageable (or device) buffer for the asynchronous snapshot copies, with MKV_E_ARG and
    nothing enqueued, whatever the Python wrapper checks; pinned memory of the same size is taken."""
    import ctypes
    torch = torch_gpu
    print("snapshot unpinned", flush=True)
    with mk.KvStore(2, 4096, F16) as a:
        fill(torch, a, 0, F16, 300, seed=830)
        fill(torch, a, 1, F16, 300, seed=831)
        nb = a.snapshot_bytes(256)
        L = mk.lib()
        for buf in (torch.zeros(nb, dtype=torch.uint8), torch.zeros(nb, dtype=torch.uint8, device="cuda")):
            for fn in (L.mkv_snapshot, L.mkv_restore):
                rc = fn(a._h, 256, ctypes.c_void_p(buf.data_ptr()), nb)
                assert rc == mk.E_ARG, (fn.__name__, rc)
                assert b"pinned" in L.mkv_last_error()
        pinned = torch.zeros(nb, dtype=torch.uint8, pin_memory=True)
        assert L.mkv_snapshot(a._h, 256, ctypes.c_void_p(pinned.data_ptr()), nb) == 0
        assert L.mkv_restore(a._h, 256, ctypes.c_void_p(pinned.data_ptr()), nb) == 0
        a.sync()
        assert a.length(0) == 256


@pytest.mark.parametrize("fmt,p", [(F16, 1000), (F16, 1024), (F32, 777), (F16, 1)])
def test_snapshot_roundtrip(torch_gpu, mk, fmt, p):
    torch = torch_gpu
    print(f"snapshot fmt={fmt} p={p}", flush=True)
    layers = 3
    q = dev(torch, q_inputs(801, 4))
    with mk.KvStore(layers, 4096, fmt) as a:
        for l in range(layers):
            fill(torch, a, l, fmt, p + 3, seed=810 + l)
        a.set_len(p)
        img = a.snapshot(p)
        assert img.numel() == a.snapshot_bytes(p)
        kn, v = kv_inputs(820, 4)
        tab = O.rope_tables(p, 4)
        outs_a = [a.append_decode(l, p + 1, dev(torch, kn), dev(torch, v), dev(torch, tab), q).cpu().numpy()
                  for l in range(layers)]
        rows_a = [caches_np(a, l, p) for l in range(layers)]
    with mk.KvStore(layers, 8192, fmt) as b:  # a fresh store, another ctx
        b.restore(p, img)
        b.sync()
        assert b.length(0) == p
        for l in range(layers):
            kb, vb = caches_np(b, l, p)
            assert np.array_equal(kb, rows_a[l][0]) and np.array_equal(vb, rows_a[l][1])
            ob = b.append_decode(l, p + 1, dev(torch, kn), dev(torch, v), dev(torch, tab), q).cpu().numpy()
            assert np.array_equal(ob, outs_a[l]), f"layer {l}: outputs differ after restore"


# ------------------------------------------------------------------------------------------------ full sizes -----

def test_decode_cfg2_full_size(torch_gpu, mk):
    """4-token verify on an f16 cache at 65,536 positions, append through the fused entry,
    then 2 drafts rolled back and the next step appended over them; both steps against the oracle."""
    torch = torch_gpu
    print("decode cfg2 full size", flush=True)
    n0, ctx = 65536, 66560
    with mk.KvStore(1, ctx, F16) as st:
        fill(torch, st, 0, F16, n0, seed=900)
        for step, pos in enumerate((n0, n0 + 2)):
            kn, v = kv_inputs(901 + step, 4)
            q = q_inputs(911 + step, 4)
            out = st.append_decode(0, pos + 1, dev(torch, kn), dev(torch, v), dev(torch, O.rope_tables(pos, 4)),
                                   dev(torch, q)).cpu().numpy()
            kc, vc = caches_np(st, 0, pos + 4)
            assert_attn_close(out, O.attn_dmx(kc, vc, q, pos + 1), what=f"cfg2 step {step}")
            st.set_len(pos + 2)  # 2 drafts rejected


def test_prefill_cfg3_all_tokens(torch_gpu, mk):
    """512 tokens appended to a cache at 28,000 positions, Q pre-scaled by 1/16 (scale 1),
    causal over 28,512 keys; every one of the 512 tokens against the oracle (about 10 s of host cores)."""
    torch = torch_gpu
    print("prefill cfg3, all tokens", flush=True)
    n0, T = 28000, 512
    with mk.KvStore(1, 28672, F16) as st:
        fill(torch, st, 0, F16, n0 + T, seed=950)
        q = q_inputs(951, T) / 16.0
        out = st.prefill(0, dev(torch, q), n0 + 1, scale=1.0).cpu().numpy()
        kc, vc = caches_np(st, 0, n0 + T)
    assert np.isfinite(out).all()
    ref = O.attn_fa_mx(kc, vc, q, n0 + 1, scale=1.0)
    assert_attn_close(out, ref, what="cfg3 prefill, 512 tokens")
    for t in (0, 255, 511):  # and per token (a bad block would hide in the Frobenius norm of the whole)
        assert_attn_close(out[t], ref[t], what=f"cfg3 prefill, token {t}")
    per_tok = np.abs(out - ref).reshape(T, -1).max(axis=1)
    assert per_tok.max() <= 2e-3, f"token {int(per_tok.argmax())}: max-abs {per_tok.max():.3e}"


def test_store_allocates_its_stated_size(torch_gpu, mk):
    """mkv_store_bytes is what mkv_create takes from the device (within the allocator's page rounding)."""
    torch = torch_gpu
    for layers, ctx, fmt in ((2, 65536, F32), (1, 4096, F16)):
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        st = mk.KvStore(layers, ctx, fmt)
        free1 = torch.cuda.mem_get_info()[0]
        st.close()
        used, stated = free0 - free1, mk.store_bytes(layers, ctx, fmt)
        assert abs(used - stated) <= 8 << 20, f"{layers} x {ctx} fmt {fmt}: took {used} B, stated {stated} B"


def seeded_fill(torch, mk, store, layer, n_pos, seed, chunk=512):
    """Large caches: seeded N(0,1) K/V generated on the device, appended through the library in chunks."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    tab = dev(torch, O.rope_tables(0, n_pos))
    for p0 in range(0, n_pos, chunk):
        m = min(chunk, n_pos - p0)
        kn = torch.randn((m, 2, 256), generator=g, device="cuda")
        v = torch.randn((m, 512), generator=g, device="cuda")
        store.append(layer, p0, kn, v, tab[p0:p0 + m])
    store.sync()


def test_decode_cfg1_full_size(torch_gpu, mk):
    """one token on an f16 cache pre-filled to 4096 positions, append of its row, attention,
    sigmoid output gate; against the oracle's attn_fd (the reference's 1-token kernel) and f64."""
    torch = torch_gpu
    print("decode cfg1 full size", flush=True)
    n0 = 4096
    with mk.KvStore(1, 8192, F16) as st:
        fill(torch, st, 0, F16, n0, seed=960)
        kn, v = kv_inputs(961, 1)
        q, qf = q_inputs(962, 1), gate_inputs(963, 1)
        out = st.append_decode(0, n0 + 1, dev(torch, kn), dev(torch, v), dev(torch, O.rope_tables(n0, 1)),
                               dev(torch, q), gate_src=dev(torch, qf)).cpu().numpy()
        kc, vc = caches_np(st, 0, n0 + 1)
    ref = O.gate(O.attn_fd(F16, kc, vc, q, n0 + 1), qf).reshape(out.shape)
    assert_attn_close(out, ref, what="cfg1 vs attn_fd + gate")
    ex = O.gate(exact_attention(kc, vc, q, n0 + 1), qf).reshape(out.shape)
    assert_attn_close(out, ex, what="cfg1 vs f64")


def test_decode_cfg4_full_size(torch_gpu, mk):
    """the 10 full-attention layers at a 262,144-position context (5.37 GB of f16 K/V), a
    4-token verify at positions 262,140..262,143 on every layer (append through the fused entry), every layer against
    the oracle, a windowed 64-token prefill on the last layer; then 2 drafts rolled back and layer 0 re-verified."""
    torch = torch_gpu
    print("decode cfg4 full size", flush=True)
    L, ctx = 10, 262144
    pos = ctx - 4
    with mk.KvStore(L, ctx, F16) as st:
        for layer in range(L):
            seeded_fill(torch, mk, st, layer, pos, seed=970 + layer)
        kn, v = kv_inputs(981, 4)
        tab = dev(torch, O.rope_tables(pos, 4))
        q = q_inputs(982, 4)
        outs = [st.append_decode(layer, pos + 1, dev(torch, kn), dev(torch, v), tab, dev(torch, q)).cpu().numpy()
                for layer in range(L)]
        assert all(np.isfinite(o).all() for o in outs)
        for layer in range(L):
            print(f"cfg4 layer {layer} vs the oracle", flush=True)
            kc, vc = caches_np(st, layer, pos + 4)
            assert_attn_close(outs[layer], O.attn_dmx(kc, vc, q, pos + 1), what=f"cfg4 layer {layer}")
        # a 64-token prefill block at the end of the last layer, over a 2,048-position window: its tiles lie more
        # than 5 GB into the store, where tile addresses have low words at and above 2^31 (the prefill kernels take
        # the tile base as a 64-bit scalar)
        T, n = 64, pos + 4 - 64 + 1
        q64 = q_inputs(985, T) / 4
        out = st.prefill(L - 1, dev(torch, q64), n, start=n - 2048).cpu().numpy()
        ref, atol, rtol = prefill_reference(F16, kc, vc, q64, n, start=n - 2048)
        assert_attn_close(out, ref, atol=atol, rtol=rtol, what="cfg4 last layer, 64-token prefill")
        st.set_len(pos + 2)
        kn2, v2 = kv_inputs(983, 2)
        q2 = q_inputs(984, 2)
        o2 = st.append_decode(0, pos + 3, dev(torch, kn2), dev(torch, v2), dev(torch, O.rope_tables(pos + 2, 2)),
                              dev(torch, q2)).cpu().numpy()
        kc, vc = caches_np(st, 0, pos + 4)
        assert_attn_close(o2, O.attn_dmx(kc, vc, q2, pos + 3), what="cfg4 after rollback")


def test_snapshot_cfg5_full_size(torch_gpu, mk):
    """f32 caches of 10 layers at 16,384 positions gathered to pinned host memory (671 MB),
    restored into a fresh store, then a 4-token verify on both: restored rows and outputs bit-identical, one layer's
    output against the oracle's f32 attn_fd."""
    torch = torch_gpu
    print("snapshot cfg5 full size", flush=True)
    L, p = 10, 16384
    kn, v = kv_inputs(991, 4)
    tab = dev(torch, O.rope_tables(p, 4))
    q = q_inputs(992, 4)
    with mk.KvStore(L, 17408, F32) as a:
        for layer in range(L):
            seeded_fill(torch, mk, a, layer, p, seed=993 + layer)
        img = a.snapshot(p)
        a.sync()
        assert img.numel() == a.snapshot_bytes(p) == L * 2 * p * 512 * 4
        assert img.is_pinned()
        rows_a = [caches_np(a, layer, p) for layer in range(L)]
        outs_a = [a.append_decode(layer, p + 1, dev(torch, kn), dev(torch, v), tab, dev(torch, q)).cpu().numpy()
                  for layer in range(L)]
        kc0, vc0 = caches_np(a, 0, p + 4)
    assert_attn_close(outs_a[0], O.attn_fd(F32, kc0, vc0, q, p + 1), atol=1e-5, rtol=1e-5, what="cfg5 f32 vs attn_fd")
    with mk.KvStore(L, 17408, F32) as b:
        b.restore(p, img)
        b.sync()
        for layer in range(L):
            kb, vb = caches_np(b, layer, p)
            assert np.array_equal(kb, rows_a[layer][0]) and np.array_equal(vb, rows_a[layer][1]), f"layer {layer}"
            ob = b.append_decode(layer, p + 1, dev(torch, kn), dev(torch, v), tab, dev(torch, q)).cpu().numpy()
            assert np.array_equal(ob, outs_a[layer]), f"layer {layer}: outputs differ after restore"


# ------------------------------------------------------------------------------------------------ root files -----

@pytest.mark.parametrize("fmt,p,background", [(F16, 1000, False), (F32, 333, True), (F16, 0, False)])
def test_root_file_roundtrip(torch_gpu, mk, tmp_path, fmt, p, background):
    """mkv_root_save writes the reference's container (parsed here independently): the tokens, the opaque state
    vectors and, per layer, K and V words of [0, p) position-major; mkv_root_load puts it into a fresh store of
    another ctx: bit-identical rows and the next verify's outputs bit-identical."""
    torch = torch_gpu
    print(f"root file fmt={fmt} p={p} background={background}", flush=True)
    layers = 3
    r = np.random.default_rng(40)
    tok = r.integers(0, 248320, p).astype(np.uint32)
    ssm = [r.standard_normal(n).astype(np.float32) for n in (64, 5)]
    conv = [r.standard_normal(n).astype(np.float32) for n in (9, 0)]
    path = tmp_path / f"root-{fmt}-{p}.bin"
    kn, v = kv_inputs(41, 4)
    tab = dev(torch, O.rope_tables(p, 4))
    q = dev(torch, q_inputs(42, 4))
    with mk.KvStore(layers, 4096, fmt) as a:
        for l in range(layers):
            fill(torch, a, l, fmt, p + 3, seed=43 + l)
        a.set_len(p)
        a.root_save(path, p, tok, ssm, conv, background=background)
        if background:
            a.root_wait()
        rows_a = [caches_np(a, l, p) for l in range(layers)]
        outs_a = [a.append_decode(l, p + 1, dev(torch, kn), dev(torch, v), tab, q).cpu().numpy()
                  for l in range(layers)]
    fp, ftok, fssm, fconv, fkv = read_root_py(path)
    assert fp == p and np.array_equal(ftok, tok) and len(fkv) == layers
    assert all(np.array_equal(x, y.view(np.uint32)) for x, y in zip(fssm + fconv, ssm + conv))
    for l in range(layers):
        for which in (0, 1):
            want = rows_a[l][which].reshape(-1)
            assert np.array_equal(fkv[l][which], want.view(np.uint32)), f"layer {l} which {which}"
    with mk.KvStore(layers, 8192, fmt) as b:
        lp, ltok, lssm, lconv = b.root_load(path)
        assert lp == p and np.array_equal(ltok, tok)
        assert all(np.array_equal(x, y) for x, y in zip(lssm + lconv, ssm + conv))
        assert all(b.length(l) == p for l in range(layers))
        for l in range(layers):
            kb, vb = caches_np(b, l, p)
            assert np.array_equal(kb, rows_a[l][0]) and np.array_equal(vb, rows_a[l][1])
            ob = b.append_decode(l, p + 1, dev(torch, kn), dev(torch, v), tab, q).cpu().numpy()
            assert np.array_equal(ob, outs_a[l]), f"layer {l}: outputs differ after the root file"
    with mk.KvStore(layers + 1, 4096, fmt) as c:  # another layer count: refused, store untouched
        with pytest.raises(mk.MkvError) as e:
            c.root_load(path)
        assert e.value.code == mk.E_FMT and c.length(0) == 0
    if p:
        with mk.KvStore(layers, 4096, 1 - fmt) as c:  # the other format: the word count does not match
            with pytest.raises(mk.MkvError) as e:
                c.root_load(path)
            assert e.value.code == mk.E_FMT


@pytest.mark.parametrize("fmt", [F32, F16])
def test_root_file_longer_than_the_staging(torch_gpu, mk, tmp_path, fmt):
    """Root saves and loads stage the position-major words in the store's prefill workspace (68 MB) in runs of
    positions, through one pinned buffer the handle keeps: 2 layers of 70,000 positions (f32: 3 runs per vector, f16:
    2) saved twice (the second save, larger, in the background, reuses and grows the buffer), loaded into a fresh
    store: rows bit-identical to the saved store's."""
    torch = torch_gpu
    print(f"root file longer than the staging fmt={fmt}", flush=True)
    layers, ctx, p = 2, 71680, 70000
    tok = np.arange(p, dtype=np.uint32)
    path = tmp_path / "big.bin"
    with mk.KvStore(layers, ctx, fmt) as a:
        for l in range(layers):
            seeded_fill(torch, mk, a, l, p, seed=60 + l)
        a.root_save(path, p - 1000, tok[:p - 1000])
        a.root_save(path, p, tok, background=True)
        a.root_wait()
        rows_a = [[a.read_rows(l, w, 0, p).clone() for w in (mk.K, mk.V)] for l in range(layers)]
    assert path.stat().st_size == 14 + 24 + 4 * p + layers * 2 * (8 + p * 512 * (4 if fmt == F32 else 2))
    with mk.KvStore(layers, ctx, fmt) as b:
        lp, ltok, _, _ = b.root_load(path)
        assert lp == p and np.array_equal(ltok, tok)
        for l in range(layers):
            for w in (mk.K, mk.V):
                assert torch.equal(b.read_rows(l, w, 0, p), rows_a[l][w]), f"layer {l} which {w}"


def test_root_file_written_like_the_reference(torch_gpu, mk, tmp_path):
    """A root file laid out by an independent writer from the oracle's f16 cache words (what read_root gathers):
    mkv_root_load puts those words into the store, and attention over them matches the oracle."""
    torch = torch_gpu
    p, layers = 700, 2
    kc = np.zeros((p + 4, 2, 256), np.uint16)
    vc = np.zeros((p + 4, 2, 256), np.uint16)
    kvw = []
    for l in range(layers):
        kcl, vcl = np.zeros_like(kc), np.zeros_like(vc)
        kn, v = kv_inputs(60 + l, p)
        O.append(F16, kcl, vcl, 0, kn, v, O.rope_tables(0, p))
        kvw.append((kcl[:p].view(np.uint32).reshape(-1), vcl[:p].view(np.uint32).reshape(-1)))
        if l == 1:
            kc, vc = kcl, vcl
    path = tmp_path / "ref.bin"
    write_root_py(path, p, np.arange(p, dtype=np.uint32), [], [], kvw)
    kn, v = kv_inputs(70, 4)
    q = q_inputs(71, 4)
    with mk.KvStore(layers, 4096, F16) as st:
        st.root_load(path)
        for l in range(layers):
            k_, v_ = caches_np(st, l, p)
            assert np.array_equal(k_.reshape(-1).view(np.uint32), kvw[l][0])
            assert np.array_equal(v_.reshape(-1).view(np.uint32), kvw[l][1])
        out = st.append_decode(1, p + 1, dev(torch, kn), dev(torch, v), dev(torch, O.rope_tables(p, 4)),
                               dev(torch, q)).cpu().numpy()
    O.append(F16, kc, vc, p, kn, v, O.rope_tables(p, 4))
    assert_attn_close(out, O.attn_dmx(kc, vc, q, p + 1), what="decode over a reference-layout root")


# ------------------------------------------------------------------------------------------------ q/k producer ---

def producer_inputs(seed, ntok):
    r = np.random.default_rng(seed)
    return (r.standard_normal((ntok, 16, 512)).astype(np.float32), r.standard_normal((ntok, 2, 256)).astype(np.float32),
            r.uniform(0.5, 1.5, 256).astype(np.float32), r.uniform(0.5, 1.5, 256).astype(np.float32))


@pytest.mark.parametrize("pos,ntok", [(0, 1), (4096, 1), (65532, 4), (1000, 512), (66000, 37), (66556, 4)])
def test_qk_norm_rope_bit_exact(torch_gpu, mk, pos, ntok):
    """The producer (rmsnorm of q and k, rope2 of q) bit-identical to the oracle's restatement, with the device
    RoPE rows bit-identical to rope_table."""
    torch = torch_gpu
    print(f"qk producer pos={pos} ntok={ntok}", flush=True)
    qf, kb, qw, kw = producer_inputs(1000 + ntok, ntok)
    with mk.KvStore(1, 66560, F16) as st:
        tab = st.rope_table_dev(pos, ntok)
        assert np.array_equal(tab.cpu().numpy(), O.rope_tables(pos, ntok))
        q, kn = st.qk_norm_rope(pos, dev(torch, qf), dev(torch, kb), dev(torch, qw), dev(torch, kw))
        q, kn = q.cpu().numpy(), kn.cpu().numpy()
    oq, okn = O.qk_norm_rope(qf, kb, qw, kw, O.rope_tables(pos, ntok))
    assert np.array_equal(kn, okn), "k norm"
    assert np.array_equal(q, oq), "q norm + rope"


def test_producer_feeds_the_verify(torch_gpu, mk):
    """producer -> fused append + decode with the device RoPE rows: the appended rows are the oracle's append of the
    oracle's normed k, the output the oracle's attn_dmx over the oracle's q."""
    torch = torch_gpu
    n0, ntok = 3000, 4
    qf, kb, qw, kw = producer_inputs(1100, ntok)
    v = np.random.default_rng(1101).standard_normal((ntok, 512)).astype(np.float32)
    with mk.KvStore(1, 4096, F16) as st:
        fill(torch, st, 0, F16, n0, seed=1102)
        q, kn = st.qk_norm_rope(n0, dev(torch, qf), dev(torch, kb), dev(torch, qw), dev(torch, kw))
        out = st.append_decode(0, n0 + 1, kn, dev(torch, v), st.rope_table_dev(n0, ntok), q).cpu().numpy()
        kc, vc = caches_np(st, 0, n0 + ntok)
    oq, okn = O.qk_norm_rope(qf, kb, qw, kw, O.rope_tables(n0, ntok))
    kc2, vc2 = kc.copy(), vc.copy()
    O.append(F16, kc2, vc2, n0, okn, v, O.rope_tables(n0, ntok))
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)
    assert_attn_close(out, O.attn_dmx(kc, vc, oq, n0 + 1), what="producer + verify")
