"""Pins the CPU oracle (oracle/mkv_oracle.c) against computations that do not share its formulas.

Function -> what pins it:
  orc_f32_to_f16     numpy's float16 cast (an independent IEEE round-to-nearest-even) on every f16 rounding boundary,
                     the midpoints between neighbours (ties), overflow, subnormals and 2^20 random bit patterns;
                     orc_f16_to_f32 on all 65536 patterns against numpy.
  orc_rope_table     th_i = pos * r^i computed by an explicit f32 recurrence in numpy; cos/sin within 1 ulp of the
                     float64 values of the same th_i (the libm routines are the reference's own choice of cosf/sinf).
  orc_append         closed forms: pos 0 (cos 1, sin 0) copies K; dims >= 64 and V are the plain f16 rounding of the
                     input; the pair (i, i+32) is rotated by th_i (norm kept, angle = th_i) within f32 rounding;
                     rotating back by -th_i recovers the input; f32 format stores the unrounded values.
  orc_attn_fd        float64 textbook softmax attention (brute force) within 1e-5; one key -> v; identical keys ->
                     mean of V; block size (16, 128, 4096) does not change the result (merge invariance).
  orc_attn_dmx       float64 brute force within the task tolerance; equal scores -> mean of the f16 V; lazy max
                     threshold exercised by a large score jump (result still within tolerance).
  orc_attn_fa_mx     float64 brute force; chunk size invariance (2048 vs 64); a selected subset of tokens equals the
                     same rows of the full call.
  orc_attn_fa_f32    float64 brute force within 1e-5.
  orc_attn_fd4       float64 brute force within 1e-5 on both formats (f32 Q: the f16-Q prefill attn_fa_mx misses that
                     bound on the same inputs); position-block size (64, 128, 512) does not change the result; one key
                     -> v; identical keys -> mean of V; a key with a large score in a later tile (the running max
                     moves and the earlier tiles are shrunk).
  orc_gate           sigmoid closed form at 0 (x/2), large positive (x), large negative (0).
  orc_gate16         numpy's float16 cast of orc_gate; ties to even, overflow to inf, subnormals.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import exact_attention, err_stats

F16, F32 = 0, 1


# ------------------------------------------------------------------------------------------------ f16 ------------

def test_f16_from_f32_matches_numpy_on_boundaries():
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = allh.view(np.float16).astype(np.float32)
    finite = np.isfinite(f)
    vals = f[finite]
    # midpoints between consecutive f16 values (ties) and values just beside them
    srt = np.unique(vals.astype(np.float64))
    mids = ((srt[:-1] + srt[1:]) / 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    extra = np.array([65504, 65519.996, 65520, 65536, 1e30, -1e30, np.inf, -np.inf, 2 ** -25, 2 ** -24, 1.5 * 2 ** -25,
                      2 ** -26, 1e-45, -0.0, 0.0, 6.1035156e-05, 6.103515e-05], np.float32)
    x = np.concatenate([vals, mids, near, extra]).astype(np.float32)
    got = O.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f16_random_bits_and_nan():
    r = np.random.default_rng(1)
    bits = r.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    assert np.array_equal(O.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16))
    nan = O.f32_to_f16_bits(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7c00) == 0x7c00 and (nan & 0x3ff) != 0


def test_f16_to_f32_all_patterns():
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    got = np.array([O.lib().orc_f16_to_f32(int(h)) for h in allh[::7]], np.float32)
    r = ref[::7]
    same = (got == r) | (np.isnan(got) & np.isnan(r))
    assert same.all()


# ------------------------------------------------------------------------------------------------ rope table -----

@pytest.mark.parametrize("pos", [0, 1, 2, 17, 4096, 65535, 65536, 262143])
def test_rope_table(pos):
    t = O.rope_table(pos)
    r = np.float32(1e7) ** np.float32(-2.0 / 64.0)
    th = np.float32(pos)
    for i in range(32):
        c64, s64 = math.cos(float(th)), math.sin(float(th))
        # within 1 ulp of the float64 value of the same f32 angle
        assert abs(t[i] - c64) <= np.spacing(np.float32(abs(c64))) + 1e-45
        assert abs(t[32 + i] - s64) <= np.spacing(np.float32(abs(s64))) + 1e-45
        th = np.float32(th * r)
    if pos == 0:
        assert np.all(t[:32] == 1.0) and np.all(t[32:] == 0.0)


# ------------------------------------------------------------------------------------------------ append ---------

def test_append_pos0_is_plain_rounding():
    r = np.random.default_rng(2)
    kn = r.standard_normal((3, 2, 256), dtype=np.float32)
    v = r.standard_normal((3, 512), dtype=np.float32)
    kc, vc = O.new_cache(4096, F16), O.new_cache(4096, F16)
    tab = np.tile(O.rope_table(0), (3, 1))  # angle 0 for all three tokens
    O.append(F16, kc, vc, 5, kn, v, tab)
    assert np.array_equal(kc[5:8], kn.astype(np.float16).view(np.uint16))
    assert np.array_equal(vc[5:8].reshape(3, 512), v.astype(np.float16).view(np.uint16))
    assert not kc[:5].any() and not kc[8:].any()


def test_append_is_a_rotation():
    r = np.random.default_rng(3)
    pos, ntok = 1000, 4
    kn = r.standard_normal((ntok, 2, 256), dtype=np.float32)
    v = r.standard_normal((ntok, 512), dtype=np.float32)
    tab = O.rope_tables(pos, ntok)
    kc, vc = O.new_cache(4096, F32), O.new_cache(4096, F32)
    O.append(F32, kc, vc, pos, kn, v, tab)
    out = kc[pos:pos + ntok].astype(np.float64)
    a = kn.astype(np.float64)
    # dims >= 64 copied exactly, V copied exactly
    assert np.array_equal(kc[pos:pos + ntok][:, :, 64:], kn[:, :, 64:])
    assert np.array_equal(vc[pos:pos + ntok].reshape(ntok, 512), v)
    rr = np.float32(1e7) ** np.float32(-2.0 / 64.0)
    for t in range(ntok):
        th = np.float32(pos + t)
        for i in range(32):
            x1, x2 = a[t, :, i], a[t, :, i + 32]
            y1, y2 = out[t, :, i], out[t, :, i + 32]
            # norm kept and angle = th_i, against float64 trigonometry of the f32 angle
            c, s = math.cos(float(th)), math.sin(float(th))
            assert np.allclose(y1, x1 * c - x2 * s, atol=1e-5)
            assert np.allclose(y2, x1 * s + x2 * c, atol=1e-5)
            assert np.allclose(np.hypot(y1, y2), np.hypot(x1, x2), rtol=1e-5)
            th = np.float32(th * rr)
    # rotating back by -th recovers the input
    back = np.array(tab)
    back[:, 32:] = -back[:, 32:]
    kc2, vc2 = O.new_cache(4096, F32), O.new_cache(4096, F32)
    O.append(F32, kc2, vc2, pos, kc[pos:pos + ntok], v, back)
    assert np.allclose(kc2[pos:pos + ntok], kn, atol=1e-5)


def test_append_f16_is_f32_then_rne():
    r = np.random.default_rng(4)
    kn = r.standard_normal((5, 2, 256), dtype=np.float32) * 100
    v = r.standard_normal((5, 512), dtype=np.float32)
    tab = O.rope_tables(777, 5)
    k16, v16 = O.new_cache(4096, F16), O.new_cache(4096, F16)
    k32, v32 = O.new_cache(4096, F32), O.new_cache(4096, F32)
    O.append(F16, k16, v16, 10, kn, v, tab)
    O.append(F32, k32, v32, 10, kn, v, tab)
    assert np.array_equal(k16[10:15], k32[10:15].astype(np.float16).view(np.uint16))
    assert np.array_equal(v16[10:15], v32[10:15].astype(np.float16).view(np.uint16))


# ------------------------------------------------------------------------------------------------ attention ------

def _cache(fmt, n, seed, ctx=4096):
    r = np.random.default_rng(seed)
    kn = r.standard_normal((n, 2, 256), dtype=np.float32)
    v = r.standard_normal((n, 512), dtype=np.float32)
    kc, vc = O.new_cache(ctx, fmt), O.new_cache(ctx, fmt)
    O.append(fmt, kc, vc, 0, kn, v, O.rope_tables(0, n))
    return kc, vc


@pytest.mark.parametrize("fmt", [F16, F32])
@pytest.mark.parametrize("n,ntok,start", [(1, 1, 0), (300, 4, 0), (1000, 1, 0), (777, 3, 100)])
def test_attn_fd_vs_f64(fmt, n, ntok, start):
    kc, vc = _cache(fmt, n + ntok - 1, 10 + n)
    q = np.random.default_rng(n).standard_normal((ntok, 16, 256), dtype=np.float32)
    got = O.attn_fd(fmt, kc, vc, q, n, start=start)
    ex = exact_attention(kc, vc, q, n, start=start)
    ma, rel = err_stats(got, ex)
    assert ma < 1e-5 and rel < 1e-5


def test_attn_fd_block_invariance():
    kc, vc = _cache(F16, 1003, 20)
    q = np.random.default_rng(21).standard_normal((4, 16, 256), dtype=np.float32)
    a = O.attn_fd(F16, kc, vc, q, 1000, bb=16)
    b = O.attn_fd(F16, kc, vc, q, 1000, bb=128)
    c = O.attn_fd(F16, kc, vc, q, 1000, bb=4096)
    assert np.allclose(a, b, atol=1e-6) and np.allclose(b, c, atol=1e-6)


def test_attn_special_cases():
    kc, vc = _cache(F16, 64, 30)
    q = np.random.default_rng(31).standard_normal((1, 16, 256), dtype=np.float32)
    v0 = O.f16_bits_to_f32(vc[0])
    # one key: out = v of position 0, for every head
    for fn in (lambda: O.attn_fd(F16, kc, vc, q, 1), lambda: O.attn_dmx(kc, vc, q, 1),
               lambda: O.attn_fa_mx(kc, vc, q, 1)):
        out = fn()
        for h in range(16):
            assert np.allclose(out[0, h], v0[h // 8], atol=1e-6)
    # identical keys: uniform weights -> mean of V
    kc2 = kc.copy()
    kc2[:50] = kc2[0]
    mean = O.f16_bits_to_f32(vc[:50]).astype(np.float64).mean(axis=0)
    for fn in (lambda: O.attn_fd(F16, kc2, vc, q, 50), lambda: O.attn_dmx(kc2, vc, q, 50),
               lambda: O.attn_fa_mx(kc2, vc, q, 50)):
        out = fn()
        for h in range(16):
            assert np.allclose(out[0, h], mean[h // 8], atol=2e-3)
    # uniform V: output = that V whatever the scores
    vc3 = vc.copy()
    vc3[:] = vc[7]
    out = O.attn_dmx(kc, vc3, q, 60)
    for h in range(16):
        assert np.allclose(out[0, h], O.f16_bits_to_f32(vc[7])[h // 8], atol=1e-3)


@pytest.mark.parametrize("n,ntok", [(1, 1), (100, 4), (2100, 4), (4093, 4), (3000, 2)])
def test_attn_dmx_vs_f64(n, ntok):
    kc, vc = _cache(F16, n + ntok - 1, 40 + n)
    q = np.random.default_rng(41 + n).standard_normal((ntok, 16, 256), dtype=np.float32)
    got = O.attn_dmx(kc, vc, q, n)
    ex = exact_attention(kc, vc, q, n)
    ma, rel = err_stats(got, ex)
    assert ma < 2e-3 and rel < 1e-3
    # f16 rounding of Q and P is really applied: not identical to the f32 path (one key: both give v exactly)
    assert n == 1 or not np.array_equal(got, O.attn_fd(F16, kc, vc, q, n))


def test_attn_dmx_lazy_max_jump():
    """A late key with a score far above the early ones moves the lazy reference max (> 8 above it)."""
    kc, vc = _cache(F16, 300, 50)
    q = np.random.default_rng(51).standard_normal((4, 16, 256), dtype=np.float32)
    # key 200 of kv head 0 parallel to q of head 0, token 0, with score q.k / 16 = 30
    c = 30 * 16 / np.dot(q[0, 0], q[0, 0])
    kc[200, 0] = (q[0, 0] * c).astype(np.float16).view(np.uint16)
    got = O.attn_dmx(kc, vc, q, 297)
    ex = exact_attention(kc, vc, q, 297)
    ma, rel = err_stats(got, ex)
    assert ma < 2e-3 and rel < 1e-3
    assert np.allclose(got[0, 0], O.f16_bits_to_f32(vc[200, 0]), atol=1e-3)  # that key dominates head 0


@pytest.mark.parametrize("n,T,start", [(2000, 64, 0), (10, 100, 0), (1500, 33, 200)])
def test_attn_fa_mx_vs_f64(n, T, start):
    kc, vc = _cache(F16, n + T - 1, 60 + T)
    q = np.random.default_rng(61 + T).standard_normal((T, 16, 256), dtype=np.float32)
    got = O.attn_fa_mx(kc, vc, q, n, start=start)
    ex = exact_attention(kc, vc, q, n, start=start)
    ma, rel = err_stats(got, ex)
    assert ma < 2e-3 and rel < 1e-3
    small = O.attn_fa_mx(kc, vc, q, n, start=start, ch=64)
    assert np.allclose(small, got, atol=1e-5)
    sel = np.array([0, T // 2, T - 1], np.int32)
    part = O.attn_fa_mx(kc, vc, q, n, start=start, sel=sel)
    assert np.array_equal(part, got[sel])


def test_attn_fa_f32_vs_f64():
    kc, vc = _cache(F32, 1000 + 40 - 1, 70)
    q = np.random.default_rng(71).standard_normal((40, 16, 256), dtype=np.float32)
    got = O.attn_fa_f32(kc, vc, q, 1000)
    ex = exact_attention(kc, vc, q, 1000)
    ma, rel = err_stats(got, ex)
    assert ma < 1e-5 and rel < 1e-5


@pytest.mark.parametrize("fmt", [F16, F32])
@pytest.mark.parametrize("n,T", [(1, 8), (1000, 32), (2047, 37), (129, 63)])
def test_attn_fd4_vs_f64(fmt, n, T):
    kc, vc = _cache(fmt, n + T - 1, 80 + T + n)
    q = np.random.default_rng(81 + T).standard_normal((T, 16, 256), dtype=np.float32)
    got = O.attn_fd4(fmt, kc, vc, q, n)
    ex = exact_attention(kc, vc, q, n)
    ma, rel = err_stats(got, ex)
    assert ma < 1e-5 and rel < 1e-5, (ma, rel)
    for bl in (128, 512):
        assert np.allclose(O.attn_fd4(fmt, kc, vc, q, n, bl=bl), got, atol=1e-6)
    if fmt == F16 and n > 1:
        # Q is not rounded to f16: the f16-Q prefill of the same block is measurably further from float64
        ma16, _ = err_stats(O.attn_fa_mx(kc, vc, q, n), ex)
        assert ma16 > 4 * ma


def test_attn_fd4_special_cases():
    kc, vc = _cache(F16, 200, 82)
    q = np.random.default_rng(83).standard_normal((8, 16, 256), dtype=np.float32)
    out = O.attn_fd4(F16, kc, vc, q, 1)  # token 0 sees one key
    v0 = O.f16_bits_to_f32(vc[0])
    for h in range(16):
        assert np.allclose(out[0, h], v0[h // 8], atol=1e-6)
    kc2 = kc.copy()
    kc2[:150] = kc2[0]  # identical keys: uniform weights, the mean of V
    out = O.attn_fd4(F16, kc2, vc, q[:1], 150)
    mean = O.f16_bits_to_f32(vc[:150]).astype(np.float64).mean(axis=0)
    for h in range(16):
        assert np.allclose(out[0, h], mean[h // 8], atol=1e-5)
    # a key in the third 64-position tile with score 40 above the rest: the running max moves past two tiles
    kc3 = kc.copy()
    c = 40 * 16 / np.dot(q[0, 3], q[0, 3])
    kc3[140, 0] = (q[0, 3] * c).astype(np.float16).view(np.uint16)
    out = O.attn_fd4(F16, kc3, vc, q, 150)
    ma, rel = err_stats(out, exact_attention(kc3, vc, q, 150))
    assert ma < 1e-5 and rel < 1e-5
    assert np.allclose(out[0, 3], O.f16_bits_to_f32(vc[140, 0]), atol=1e-5)


def test_gate_closed_form():
    att = np.random.default_rng(80).standard_normal((2, 16, 256), dtype=np.float32)
    qf = np.zeros((2, 16, 512), np.float32)
    assert np.allclose(O.gate(att, qf), att.reshape(2, -1) / 2)
    qf[:, :, 256:] = 100.0
    assert np.allclose(O.gate(att, qf), att.reshape(2, -1))
    qf[:, :, 256:] = -100.0
    assert np.allclose(O.gate(att, qf), 0.0, atol=1e-30)
    qf[:, :, :256] = 1e9  # the q half of qf is not read
    assert np.allclose(O.gate(att, qf), 0.0, atol=1e-30)


def test_gate16_rounds_the_f32_gate_to_nearest_even():
    """attn_gate16 (ops.wgsl:296-300) = pack2x16float of attn_gate's f32 product: numpy's float16 cast (round to
    nearest even) of orc_gate's output, exact ties to even, overflow to infinity, subnormals kept."""
    rng = np.random.default_rng(81)
    att = rng.standard_normal((3, 16, 256), dtype=np.float32)
    qf = rng.standard_normal((3, 16, 512), dtype=np.float32)
    want = O.gate(att, qf).astype(np.float16).view(np.uint16)
    assert np.array_equal(O.gate16(att, qf), want)
    # sigmoid(100) is 1 in f32, so the output is f16(att): ties and range edges
    qf[:] = 100.0
    att = np.zeros((1, 16, 256), np.float32)
    att.flat[:6] = [1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, -(1 + 2.0 ** -11), 70000.0, -70000.0, 2.0 ** -20]
    got = O.gate16(att, qf[:1]).ravel()[:6]
    assert list(got) == [0x3C00, 0x3C02, 0xBC00, 0x7C00, 0xFC00, 0x0010]


# ---- q/k producer: rmsnorm (ops.wgsl:27-57) and rope2 (ops.wgsl:275-286) ----

def test_rmsnorm_closed_forms():
    w = np.ones(256, np.float32)
    for c in (1.0, 2.0, 0.5, -4.0):  # constant rows, eps 0: sum = 256 c^2, scale = 1/|c| exactly
        y = O.rmsnorm_rows(np.full(256, c, np.float32), w, eps=0.0)
        assert np.array_equal(y[0], np.full(256, math.copysign(1.0, c), np.float32))
    x = np.random.default_rng(90).standard_normal(256).astype(np.float32)
    assert np.array_equal(O.rmsnorm_rows(x, 2 * w)[0], 2 * O.rmsnorm_rows(x, w)[0])  # the weight is a last product


def test_rmsnorm_is_the_256_thread_tree():
    # x[1]^2 + x[129]^2 meet first in the reference's tree (m = 128), then join 2^24: the sum is 2^24 + 2 exactly,
    # where a running sum would round 2^24 + 1 back to 2^24 twice
    x = np.zeros(256, np.float32)
    x[0], x[1], x[129] = 4096.0, 1.0, 1.0
    w = np.random.default_rng(91).uniform(0.5, 1.5, 256).astype(np.float32)
    s = np.float32(2**24 + 2)
    scale = np.float32(1.0) / np.sqrt(s / np.float32(256.0) + np.float32(1e-6))  # IEEE f32 ops
    assert np.array_equal(O.rmsnorm_rows(x, w, eps=1e-6)[0], (x * scale) * w)
    run = np.float32(0)
    for v in x:
        run = np.float32(run + v * v)
    assert run == np.float32(2**24)  # the sequential order would differ


def test_rmsnorm_vs_float64():
    r = np.random.default_rng(92)
    x = (r.standard_normal((64, 256)) * r.uniform(1e-3, 1e3, (64, 1))).astype(np.float32)
    w = r.uniform(0.5, 1.5, 256).astype(np.float32)
    y = O.rmsnorm_rows(x, w, eps=1e-6)
    x64 = x.astype(np.float64)
    ex = x64 / np.sqrt((x64 * x64).mean(1, keepdims=True) + 1e-6) * w
    assert np.abs(y - ex).max() <= 3e-7 * np.abs(ex).max()
    # rows at a stride (q rows of qf: 256 q values then 256 gate values)
    qf = r.standard_normal((3, 512)).astype(np.float32)
    assert np.array_equal(O.rmsnorm_rows(qf, w, step=512), O.rmsnorm_rows(qf[:, :256], w))


def test_qk_norm_rope_position_zero_and_rotation():
    r = np.random.default_rng(93)
    ntok = 3
    qf = r.standard_normal((ntok, 16, 512)).astype(np.float32)
    kb = r.standard_normal((ntok, 2, 256)).astype(np.float32)
    qw = r.uniform(0.5, 1.5, 256).astype(np.float32)
    kw = r.uniform(0.5, 1.5, 256).astype(np.float32)
    qn = O.rmsnorm_rows(qf.reshape(-1), qw, step=512).reshape(ntok, 16, 256)
    q0, k0 = O.qk_norm_rope(qf, kb, qw, kw, np.tile(O.rope_table(0), (ntok, 1)))
    assert np.array_equal(q0, qn)  # cos 0 = 1, sin 0 = 0: no rotation (x*1 - y*0 is exact)
    assert np.array_equal(k0, O.rmsnorm_rows(kb.reshape(-1), kw).reshape(ntok, 2, 256))
    pos = 5000
    tab = O.rope_tables(pos, ntok)
    q1, k1 = O.qk_norm_rope(qf, kb, qw, kw, tab)
    assert np.array_equal(k1, k0)  # k is not rotated here (the append rotates it)
    assert np.array_equal(q1[:, :, 64:], qn[:, :, 64:])
    a, b = qn[:, :, :32].astype(np.float64), qn[:, :, 32:64].astype(np.float64)
    c, s = tab[:, None, :32].astype(np.float64), tab[:, None, 32:].astype(np.float64)
    assert np.allclose(q1[:, :, :32], a * c - b * s, atol=1e-6)  # rotation of each pair (i, i + 32) by th_i
    assert np.allclose(q1[:, :, 32:64], a * s + b * c, atol=1e-6)
