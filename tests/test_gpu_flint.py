"""GPU parity tests of the Flint KV path (include/mechta_flint.h) through the C ABI, against the CPU oracle
(oracle/flint_oracle.c).

Bars: ring writes, row conversion, RoPE and photo bit-exact; attention (f32-class arithmetic on f32 or f16 caches, as
the reference's f32: f16 matrix products of split f32 operands) within max-abs 1e-5 and relative (Frobenius) 1e-5 of attn_fd + attn_fd_merge (one token) or attn_pf (a
block), with sinks, windows and ring wraps.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_attn_close

pytestmark = pytest.mark.gpu

F16, F32 = 0, 1
H, KVH, D = 32, 4, 128
TOL = 1e-5


@pytest.fixture(scope="module")
def mf(torch_gpu):
    from mechta_amd import flint
    flint.lib()
    return flint


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rng(seed):
    return np.random.default_rng(seed)


def fill(torch, st, kc, vc, layer, fmt, pos1, seed, block=512):
    """Positions [0, pos1) appended in blocks through the GPU store and the oracle's caches alike."""
    r = rng(seed)
    p = 0
    while p < pos1:
        n = min(block, pos1 - p)
        k = r.standard_normal((n, KVH, D), dtype=np.float32)
        v = r.standard_normal((n, KVH, D), dtype=np.float32)
        st.append(layer, p, dev(torch, k), dev(torch, v))
        O.fl_kv_write(fmt, kc, vc, p, k, v)
        p += n


def rows_np(st, layer, which):
    x = st.read_rows(layer, which, 0, st.rows(layer)).cpu().numpy()
    return x.view(np.uint16) if x.dtype == np.int16 else x


@pytest.mark.parametrize("fmt", [F32, F16])
def test_append_ring_bit_exact(torch_gpu, mf, fmt):
    torch = torch_gpu
    with mf.FlintStore(2, 4096, fmt, sliding=[True, False]) as st:
        for layer in (0, 1):
            rows = st.rows(layer)
            assert rows == (1024 if layer == 0 else 4096)
            kc, vc = O.fl_new_cache(rows, fmt), O.fl_new_cache(rows, fmt)
            fill(torch, st, kc, vc, layer, fmt, 2900, seed=1 + layer, block=333)  # wraps the ring twice
            assert np.array_equal(rows_np(st, layer, 0), kc) and np.array_equal(rows_np(st, layer, 1), vc)


@pytest.mark.parametrize("fmt", [F32, F16])
def test_rows_roundtrip_and_photo(torch_gpu, mf, fmt):
    torch = torch_gpu
    with mf.FlintStore(3, 2048, fmt, sliding=[True, False, True]) as st:
        kc, vc = O.fl_new_cache(1024, fmt), O.fl_new_cache(1024, fmt)
        fill(torch, st, kc, vc, 0, fmt, 1500, seed=3)
        st.photo()
        k0, v0 = rows_np(st, 0, 0), rows_np(st, 0, 1)
        kc2, vc2 = kc.copy(), vc.copy()
        fill(torch, st, kc2, vc2, 0, fmt, 1700, seed=4)  # overwrites the ring
        assert not np.array_equal(rows_np(st, 0, 0), k0)
        st.restore_photo()
        assert np.array_equal(rows_np(st, 0, 0), k0) and np.array_equal(rows_np(st, 0, 1), v0)
        # rows written in the reference layout come back unchanged (a root's words)
        src = rows_np(st, 0, 1)[100:300]
        st.write_rows(2, 1, 0, 200, dev(torch, src.view(np.int16) if fmt == F16 else src))
        assert np.array_equal(rows_np(st, 2, 1)[:200], src)


def test_rope_bit_exact(torch_gpu, mf):
    torch = torch_gpu
    x = rng(5).standard_normal((7, H, D), dtype=np.float32)
    tabs = O.fl_rope_tables(1234, 7)
    with mf.FlintStore(1, 1024, F32, sliding=[True]) as st:
        y = st.rope(dev(torch, x), dev(torch, tabs)).cpu().numpy()
    assert np.array_equal(y, O.fl_rope(x, tabs))


# (fmt, sliding, ctx, pos): one token at pos, after positions [0, pos] were written
DECODE = [(F32, False, 4096, 3000), (F16, False, 4096, 777), (F32, True, 4096, 2500), (F16, True, 4096, 1100),
          (F32, True, 4096, 100), (F32, False, 40960, 40000), (F16, False, 40960, 32768), (F32, False, 4096, 0),
          (F16, True, 8192, 5000), (F16, False, 4096, 4095), (F32, False, 4096, 4095),  # these two: ctx's last row
          # either side of the spans whose decode merges in the kernel (f32 up to 384 positions, f16 up to 512)
          (F32, False, 4096, 383), (F32, False, 4096, 384), (F16, False, 4096, 300), (F16, False, 4096, 511),
          (F16, False, 4096, 512)]


@pytest.mark.parametrize("fmt,sliding,ctx,pos", DECODE)
def test_decode_vs_attn_fd(torch_gpu, mf, fmt, sliding, ctx, pos):
    torch = torch_gpu
    print(f"flint decode fmt={fmt} sliding={sliding} pos={pos}", flush=True)
    win = 513 if sliding else 0
    with mf.FlintStore(1, ctx, fmt, sliding=[sliding]) as st:
        kc, vc = O.fl_new_cache(st.rows(0), fmt), O.fl_new_cache(st.rows(0), fmt)
        fill(torch, st, kc, vc, 0, fmt, pos + 1, seed=10 + pos)
        q = rng(11).standard_normal((1, H, D), dtype=np.float32)
        sinks = rng(12).standard_normal(H, dtype=np.float32)
        out = st.attend(0, pos, dev(torch, q), dev(torch, sinks)).cpu().numpy()
    ref = O.fl_attn_fd(fmt, kc, vc, q[0], pos, win, sinks)
    assert_attn_close(out[0], ref, atol=TOL, rtol=TOL, what="flint decode vs attn_fd")


# (fmt, sliding, ctx, pos0, T)
PREFILL = [(F32, False, 4096, 200, 70), (F16, False, 4096, 0, 9), (F32, True, 4096, 1900, 40), (F16, True, 4096, 600, 33),
           (F32, True, 8192, 5000, 512), (F16, False, 8192, 3000, 512), (F32, False, 4096, 0, 512), (F16, True, 4096, 3, 5),
           (F32, True, 4096, 2000, 2), (F16, False, 8192, 5000, 2), (F32, False, 4096, 1000, 3), (F16, True, 4096, 1500, 4),
           (F32, False, 40960, 39000, 2), (F16, True, 8192, 5000, 512), (F16, True, 4096, 1037, 100),
           (F16, False, 40960, 39000, 257), (F16, False, 4096, 31, 63), (F16, False, 40960, 30000, 8),
           (F32, False, 40960, 30001, 12), (F16, True, 40960, 30002, 29),
           (F16, False, 4096, 3584, 512), (F32, False, 4096, 4092, 4), (F16, False, 4096, 4094, 2),  # up to ctx's end
           (F16, False, 4096, 200, 2), (F32, False, 4096, 100, 2)]  # two tokens merged in the kernel (short spans)


@pytest.mark.parametrize("fmt,sliding,ctx,pos0,T", PREFILL)
def test_prefill_vs_attn_pf(torch_gpu, mf, fmt, sliding, ctx, pos0, T):
    torch = torch_gpu
    print(f"flint prefill fmt={fmt} sliding={sliding} pos0={pos0} T={T}", flush=True)
    win = 513 if sliding else 0
    with mf.FlintStore(1, ctx, fmt, sliding=[sliding]) as st:
        kc, vc = O.fl_new_cache(st.rows(0), fmt), O.fl_new_cache(st.rows(0), fmt)
        fill(torch, st, kc, vc, 0, fmt, pos0 + T, seed=20 + pos0)
        q = rng(21).standard_normal((T, H, D), dtype=np.float32)
        sinks = rng(22).standard_normal(H, dtype=np.float32)
        out = st.attend(0, pos0, dev(torch, q), dev(torch, sinks)).cpu().numpy()
    ref = O.fl_attn_pf(fmt, kc, vc, q, pos0, win, sinks)
    assert_attn_close(out, ref, atol=TOL, rtol=TOL, what="flint prefill vs attn_pf")


def test_no_sinks(torch_gpu, mf):
    torch = torch_gpu
    with mf.FlintStore(1, 4096, F32, sliding=[False]) as st:
        kc, vc = O.fl_new_cache(4096, F32), O.fl_new_cache(4096, F32)
        fill(torch, st, kc, vc, 0, F32, 1300, seed=30)
        q = rng(31).standard_normal((1, H, D), dtype=np.float32)
        out = st.attend(0, 1299, dev(torch, q)).cpu().numpy()
    assert_attn_close(out[0], O.fl_attn_fd(F32, kc, vc, q[0], 1299, 0, None), atol=TOL, rtol=TOL, what="no sinks")


@pytest.mark.parametrize("fmt", [F32, F16])
def test_nan_rows_outside_the_window(torch_gpu, mf, fmt):
    """Ring rows of positions outside every token's window, and full-layer rows past the block, may hold anything
    (NaN included): decode and prefill keep them out."""
    torch = torch_gpu
    pos0, T = 3000, 64
    with mf.FlintStore(2, 4096, fmt, sliding=[True, False]) as st:
        caches = []
        for layer in (0, 1):
            kc, vc = O.fl_new_cache(st.rows(layer), fmt), O.fl_new_cache(st.rows(layer), fmt)
            fill(torch, st, kc, vc, layer, fmt, pos0 + T, seed=40 + layer)
            caches.append((kc, vc))
        nan = np.full((1, KVH, D), np.nan, np.float32)
        if fmt == F16:
            nan = nan.astype(np.float16).view(np.int16)
        hidden = sorted({p % 1024 for p in range(pos0 + T - 1024, pos0 - 512)})  # sliding: before every window
        for r in hidden[::7]:
            for which in (0, 1):
                st.write_rows(0, which, r, r + 1, dev(torch, nan))
        for r in range(pos0 + T, pos0 + T + 40):  # full layer: past the block
            for which in (0, 1):
                st.write_rows(1, which, r, r + 1, dev(torch, nan))
        q = rng(43).standard_normal((T, H, D), dtype=np.float32)
        sinks = rng(44).standard_normal(H, dtype=np.float32)
        for layer, win in ((0, 513), (1, 0)):
            kc, vc = caches[layer]
            outp = st.attend(layer, pos0, dev(torch, q), dev(torch, sinks)).cpu().numpy()
            assert_attn_close(outp, O.fl_attn_pf(fmt, kc, vc, q, pos0, win, sinks), atol=TOL, rtol=TOL,
                              what=f"prefill layer {layer} next to NaN rows")
            outd = st.attend(layer, pos0 + T - 1, dev(torch, q[-1:]), dev(torch, sinks)).cpu().numpy()
            assert_attn_close(outd[0], O.fl_attn_fd(fmt, kc, vc, q[-1], pos0 + T - 1, win, sinks), atol=TOL,
                              rtol=TOL, what=f"decode layer {layer} next to NaN rows")


@pytest.mark.parametrize("fmt", [F32, F16])
def test_captured_step_replay_bit_identical(torch_gpu, mf, fmt):
    """A Flint step under HIP graph capture (the reference records its commands once, flint.rs builds them per step
    shape): ring append of a 64-token block and its prefill attention on a sliding and a full layer, then a one-token
    decode on each. Attention and append allocate nothing after create, so no eager call precedes the capture. Every
    replay equals the eager step bit for bit (replays re-append the same rows), with eager attention of the same
    store between replays."""
    torch = torch_gpu
    print(f"flint graph capture fmt={fmt}", flush=True)
    pos0, T = 1500, 64
    with mf.FlintStore(2, 4096, fmt, sliding=[True, False]) as st:
        for layer in (0, 1):
            kc, vc = O.fl_new_cache(st.rows(layer), fmt), O.fl_new_cache(st.rows(layer), fmt)
            fill(torch, st, kc, vc, layer, fmt, pos0, seed=50 + layer)
        r = rng(52)
        k, v = (dev(torch, r.standard_normal((T, KVH, D), dtype=np.float32)) for _ in range(2))
        q = dev(torch, r.standard_normal((T, H, D), dtype=np.float32))
        q1 = dev(torch, r.standard_normal((1, H, D), dtype=np.float32))
        sinks = dev(torch, r.standard_normal(H, dtype=np.float32))

        def step(outs):
            for layer in (0, 1):
                st.append(layer, pos0, k, v)
                st.attend(layer, pos0, q, sinks, out=outs[2 * layer])
                st.attend(layer, pos0 + T - 1, q1, sinks, out=outs[2 * layer + 1])

        shapes = [(T, H, D), (1, H, D)] * 2
        eager = [torch.empty(s, dtype=torch.float32, device="cuda") for s in shapes]
        step(eager)
        torch.cuda.synchronize()
        outs = [torch.empty_like(x) for x in eager]
        g = torch.cuda.CUDAGraph()
        base_stream = torch.cuda.current_stream()
        with torch.cuda.graph(g):
            st.set_stream(torch.cuda.current_stream())
            step(outs)
        st.set_stream(base_stream)
        torch.cuda.synchronize()
        for rep in range(4):
            for x in outs:
                x.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(outs, eager)):
                assert torch.equal(a, b), f"replay {rep}: output {i} differs from the eager step"
            st.attend(1, 700, q1, sinks)  # eager work of the same store between replays
            st.attend(0, pos0 - 1, q, sinks)
            torch.cuda.synchronize()


@pytest.mark.parametrize("fmt", [F32, F16])
@pytest.mark.parametrize("seed", [1, 2])
def test_random_call_sequence(torch_gpu, mf, fmt, seed):
    """A seeded sequence of ragged appends to a full and a sliding layer in step, with attention calls of 1 to 130
    tokens ending at the written length on either layer in between (the sliding ring wraps several times): every
    output against the oracle's attn_fd / attn_pf on its own caches fed the same appends, and the rings end
    bit-identical."""
    torch = torch_gpu
    r = rng(500 + 10 * seed + fmt)
    ctx = 8192
    with mf.FlintStore(2, ctx, fmt, sliding=[False, True]) as st:
        caches = [(O.fl_new_cache(st.rows(layer), fmt), O.fl_new_cache(st.rows(layer), fmt)) for layer in range(2)]
        sinks = r.standard_normal(H, dtype=np.float32)
        pos = 0
        for step in range(40):
            if pos < 600 or (r.random() < 0.4 and pos < ctx - 300):
                m = int(r.integers(1, 300))
                k = r.standard_normal((m, KVH, D), dtype=np.float32)
                v = r.standard_normal((m, KVH, D), dtype=np.float32)
                for layer in range(2):
                    st.append(layer, pos, dev(torch, k), dev(torch, v))
                    O.fl_kv_write(fmt, caches[layer][0], caches[layer][1], pos, k, v)
                pos += m
                continue
            layer = int(r.integers(0, 2))
            T = int(r.choice([1, 2, 3, 4, 8, 33, 64, 100, 130]))
            pos0 = pos - T
            print(f"flint sequence fmt={fmt} seed={seed} step {step}: layer {layer} T={T} pos0={pos0}", flush=True)
            q = r.standard_normal((T, H, D), dtype=np.float32)
            out = st.attend(layer, pos0, dev(torch, q), dev(torch, sinks)).cpu().numpy()
            kc, vc = caches[layer]
            win = 513 if layer == 1 else 0
            ref = O.fl_attn_fd(fmt, kc, vc, q[0], pos0, win, sinks)[None] if T == 1 else \
                O.fl_attn_pf(fmt, kc, vc, q, pos0, win, sinks)
            assert_attn_close(out.reshape(ref.shape), ref, atol=TOL, rtol=TOL,
                              what=f"step {step} layer {layer} T={T}")
        for layer in range(2):
            for which in range(2):
                assert np.array_equal(rows_np(st, layer, which).reshape(-1),
                                      caches[layer][which].reshape(-1)), f"layer {layer} plane {which} differs"
