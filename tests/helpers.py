"""Shared helpers of the tests: seeded inputs, tolerance checks, GPU <-> oracle plumbing."""
import numpy as np

from oracle import oracle as O

H, KVH, D = 16, 2, 256

# attention tolerance of the task (north star): max-abs 2e-3 and relative (Frobenius) 1e-3 against the oracle
ATOL, RTOL = 2e-3, 1e-3


def rng(seed):
    return np.random.default_rng(seed)


def kv_inputs(seed, ntok):
    """Seeded N(0,1) f32 inputs of an append of ntok tokens: k_normed [ntok][2][256], v [ntok][512]."""
    r = rng(seed)
    return (r.standard_normal((ntok, KVH, D), dtype=np.float32),
            r.standard_normal((ntok, KVH * D), dtype=np.float32))


def q_inputs(seed, ntok):
    r = rng(seed)
    return r.standard_normal((ntok, H, D), dtype=np.float32)


def gate_inputs(seed, ntok):
    r = rng(seed)
    return r.standard_normal((ntok, H, 512), dtype=np.float32)


def err_stats(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    max_abs = float(np.abs(got - ref).max())
    rel = float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))
    return max_abs, rel


def assert_attn_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    max_abs, rel = err_stats(got, ref)
    assert max_abs <= atol and rel <= rtol, f"{what}: max-abs {max_abs:.3e} (tol {atol}), rel {rel:.3e} (tol {rtol})"
    return max_abs, rel


SMALL_PREFILL_MAX = 63  # f16 blocks up to this many tokens run f32-class, as the reference's attn_fd4


def prefill_reference(fmt, kc, vc, q, n0, start=0, sel=None):
    """(reference rows, atol, rtol) of a prefill of the block q: the oracle function of the reference kernel the block
    takes (engine.rs:1215-1241) and the bar it is held to. f32 store: attn_fa (exact f32), 1e-5; f16 store, blocks of
    64 tokens or more: attn_fa_mx, the task tolerance; f16 blocks under 64 tokens: attn_fd4 (f32 Q, exact max; with a
    window start, attn_fd per token, the same f32 arithmetic), 1e-5."""
    T = np.asarray(q).reshape(-1, H, D).shape[0]
    if sel is None:
        sel = np.arange(T, dtype=np.int32)
    if fmt == 1:
        return O.attn_fa_f32(kc, vc, q, n0, start=start, sel=sel), 1e-5, 1e-5
    if T > SMALL_PREFILL_MAX:
        return O.attn_fa_mx(kc, vc, q, n0, start=start, sel=sel), ATOL, RTOL
    full = O.attn_fd4(0, kc, vc, q, n0) if start == 0 else O.attn_fd(0, kc, vc, q, n0, start=start)
    return full[sel], 1e-5, 1e-5


def exact_attention(kc, vc, q, n, start=0, scale=1.0 / 16):
    """Textbook softmax attention in float64 (brute force), reference layout caches; token t sees [start, n + t)."""
    K = O.f16_bits_to_f32(kc) if kc.dtype == np.uint16 else kc
    V = O.f16_bits_to_f32(vc) if vc.dtype == np.uint16 else vc
    K = K.astype(np.float64)
    V = V.astype(np.float64)
    q = np.asarray(q, np.float64).reshape(-1, H, D)
    out = np.empty(q.shape)
    for t in range(q.shape[0]):
        e = n + t
        for h in range(H):
            s = K[start:e, h // 8] @ q[t, h] * scale
            w = np.exp(s - s.max())
            out[t, h] = (w @ V[start:e, h // 8]) / w.sum()
    return out


# ---- root files (session.rs:92-129), written and parsed here independently of the library ----

ROOT_HEADER = b"MECHTA-ROOT-1\n"


def fnv1a64(data: bytes) -> int:
    """FNV-1a 64 (Fowler/Noll/Vo): offset basis 0xcbf29ce484222325, prime 0x100000001b3, per byte xor then multiply."""
    x = 0xCBF29CE484222325
    for b in data:
        x = ((x ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return x


def write_root_py(path, p, tokens, ssm, conv, kv):
    """A root file as write_root_file lays it out: header, u64 p, ns, nk, u32 tokens, ssm vectors, conv vectors,
    (K, V) vectors; vector = u64 word count + the words (kv: list of (K words, V words), 32-bit arrays)."""
    import struct
    with open(path, "wb") as f:
        f.write(ROOT_HEADER)
        f.write(struct.pack("<QQQ", p, len(ssm), len(kv)))
        f.write(np.asarray(tokens, "<u4").tobytes())
        for vecs in (ssm, conv):
            for a in vecs:
                a = np.ascontiguousarray(a).view("<u4")
                f.write(struct.pack("<Q", a.size))
                f.write(a.tobytes())
        for k, v in kv:
            for a in (k, v):
                a = np.ascontiguousarray(a).view("<u4")
                f.write(struct.pack("<Q", a.size))
                f.write(a.tobytes())


def read_root_py(path):
    """Parses a root file like read_root_file: (p, tokens, ssm, conv, kv) with 32-bit word arrays (uint32)."""
    import struct
    b = open(path, "rb").read()
    assert b.startswith(ROOT_HEADER)
    o = len(ROOT_HEADER)
    p, ns, nk = struct.unpack_from("<QQQ", b, o)
    o += 24
    tokens = np.frombuffer(b, "<u4", p, o)
    o += 4 * p

    def vec():
        nonlocal o
        (n,) = struct.unpack_from("<Q", b, o)
        o += 8
        a = np.frombuffer(b, "<u4", n, o)
        o += 4 * n
        return a

    ssm = [vec() for _ in range(ns)]
    conv = [vec() for _ in range(ns)]
    kv = [(vec(), vec()) for _ in range(nk)]
    assert o == len(b), "trailing bytes"
    return p, tokens, ssm, conv, kv
