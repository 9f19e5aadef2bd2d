"""Writes tests/golden/fixtures.npz: small input/output vectors of the KV-cache path, computed by the CPU oracle.

The reference ships no golden vectors for this path and cannot run here (Rust + WGSL through wgpu/Vulkan), so these
fixtures are regression vectors of the oracle restatement: tests/test_golden.py checks that the oracle still
reproduces them (CPU) and that the HIP path matches them through the C ABI (GPU). Inputs are not stored: they come
from `normals(seed, n)` below, a documented counter-based generator (SplitMix64 finalizer on seed and index, two
53-bit uniforms, Box-Muller), so the GPU box rebuilds them bit for bit without numpy's generator streams. The first
values of each input stream are stored to pin the generator itself.

Cases (positions 0-based; token t of a step at position pos sees [start, pos + 1 + t)):
  append4_f16   300 prefix rows, then 4 rows at 300: the 4 appended K/V rows (f16 bits) and a SHA-256 of every row
  decode4_f16   4-token verify at n = 301 over that cache: attn_dmx (dmx.rs:19-138)
  decode1_gate  1 token at n = 1001 over 1001 rows, sigmoid output gate: attn_fd + attn_gate (ops.wgsl:310-394, 171-177)
  prefill64     64 tokens at n = 2001 over 2000 + 64 rows: attn_fa_mx (fa_mx.wgsl:19-115), 4 sampled tokens
  rows_f32      3 f32 layers x 256 rows: SHA-256 of each layer's K and V words (read_root order, engine.rs:782-823)
  flint_full    Flint, f32 full layer, 300 rows, token at 299 with sinks: attn_fd + attn_fd_merge (flint_attn.wgsl)
  flint_slide   Flint, f16 sliding layer (ring 1024, window 513), 1500 rows (a ring wrap), token at 1499, sinks

Run from the repository root: python -m tests.golden.gen_fixtures
"""
import hashlib
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "fixtures.npz")
M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _mix(z):
    """SplitMix64 finalizer (Steele, Lea, Flood 2014), on uint64 arrays (wrapping arithmetic)."""
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def normals(seed, shape):
    """N(0,1) float32 values: element i uses x_k = mix(seed * 2^32 + 2i + k) for k = 0, 1; u_k = ((x_k >> 11) + 1)
    * 2^-53 in (0, 1]; value = float32(sqrt(-2 ln u_0) cos(2 pi u_1)) computed in float64."""
    n = int(np.prod(shape))
    i = np.arange(n, dtype=np.uint64)
    base = np.uint64(seed) << np.uint64(32)
    with np.errstate(over="ignore"):
        x0 = _mix(base + np.uint64(2) * i)
        x1 = _mix(base + np.uint64(2) * i + np.uint64(1))
    u0 = ((x0 >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u1 = ((x1 >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    return (np.sqrt(-2.0 * np.log(u0)) * np.cos(2.0 * np.pi * u1)).astype(np.float32).reshape(shape)


def sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), np.uint8)


# seeds of the input streams, by case
SEEDS = dict(prefix=101, new4=102, q4=103, prefix1k=111, new1=112, q1=113, gate1=114, prefix2k=121, new64=122,
             q64=123, f32rows=131, fl_full=141, fl_full_q=142, fl_sinks=143, fl_slide=151, fl_slide_q=152)
PF_SEL = np.array([0, 17, 40, 63], np.int32)


def inputs():
    """Every input array of the cases, from the seeds above."""
    H, KVH, D = 16, 2, 256
    x = {}
    x["kn300"], x["v300"] = normals(SEEDS["prefix"], (300, KVH, D)), normals(SEEDS["prefix"] + 1000, (300, KVH * D))
    x["kn4"], x["v4"] = normals(SEEDS["new4"], (4, KVH, D)), normals(SEEDS["new4"] + 1000, (4, KVH * D))
    x["q4"] = normals(SEEDS["q4"], (4, H, D))
    x["kn1k"], x["v1k"] = normals(SEEDS["prefix1k"], (1000, KVH, D)), normals(SEEDS["prefix1k"] + 1000, (1000, KVH * D))
    x["kn1"], x["v1"] = normals(SEEDS["new1"], (1, KVH, D)), normals(SEEDS["new1"] + 1000, (1, KVH * D))
    x["q1"], x["gate1"] = normals(SEEDS["q1"], (1, H, D)), normals(SEEDS["gate1"], (1, H, 512))
    x["kn2k"], x["v2k"] = normals(SEEDS["prefix2k"], (2000, KVH, D)), normals(SEEDS["prefix2k"] + 1000, (2000, KVH * D))
    x["kn64"], x["v64"] = normals(SEEDS["new64"], (64, KVH, D)), normals(SEEDS["new64"] + 1000, (64, KVH * D))
    x["q64"] = normals(SEEDS["q64"], (64, H, D)) / np.float32(16.0)
    x["f32rows"] = [(normals(SEEDS["f32rows"] + 10 * l, (256, KVH, D)), normals(SEEDS["f32rows"] + 10 * l + 5, (256, KVH * D)))
                    for l in range(3)]
    FH, FKVH, FD = 32, 4, 128
    x["fl_full_k"], x["fl_full_v"] = normals(SEEDS["fl_full"], (300, FKVH, FD)), normals(SEEDS["fl_full"] + 1000, (300, FKVH, FD))
    x["fl_full_q"] = normals(SEEDS["fl_full_q"], (FH, FD))
    x["fl_sinks"] = normals(SEEDS["fl_sinks"], (FH,))
    x["fl_slide_k"] = normals(SEEDS["fl_slide"], (1500, FKVH, FD))
    x["fl_slide_v"] = normals(SEEDS["fl_slide"] + 1000, (1500, FKVH, FD))
    x["fl_slide_q"] = normals(SEEDS["fl_slide_q"], (FH, FD))
    return x


def expected(x):
    """The oracle's outputs for every case (CPU; oracle/ is test infrastructure)."""
    from oracle import oracle as O
    e = {}
    # append4_f16 / decode4_f16
    kc, vc = O.new_cache(4096, 0), O.new_cache(4096, 0)
    O.append(0, kc, vc, 0, x["kn300"], x["v300"], O.rope_tables(0, 300))
    O.append(0, kc, vc, 300, x["kn4"], x["v4"], O.rope_tables(300, 4))
    e["append4_k"], e["append4_v"] = kc[300:304].copy(), vc[300:304].copy()
    e["append4_sha_k"], e["append4_sha_v"] = sha(kc[:304]), sha(vc[:304])
    e["decode4"] = O.attn_dmx(kc, vc, x["q4"], 301)
    # decode1_gate
    kc, vc = O.new_cache(4096, 0), O.new_cache(4096, 0)
    O.append(0, kc, vc, 0, x["kn1k"], x["v1k"], O.rope_tables(0, 1000))
    O.append(0, kc, vc, 1000, x["kn1"], x["v1"], O.rope_tables(1000, 1))
    e["decode1_gate"] = O.gate(O.attn_fd(0, kc, vc, x["q1"], 1001), x["gate1"]).reshape(1, 16, 256)
    # prefill64
    kc, vc = O.new_cache(4096, 0), O.new_cache(4096, 0)
    O.append(0, kc, vc, 0, x["kn2k"], x["v2k"], O.rope_tables(0, 2000))
    O.append(0, kc, vc, 2000, x["kn64"], x["v64"], O.rope_tables(2000, 64))
    e["prefill64"] = O.attn_fa_mx(kc, vc, x["q64"], 2001, scale=1.0, sel=PF_SEL)
    # rows_f32
    shas = []
    for kn, v in x["f32rows"]:
        kc, vc = O.new_cache(4096, 1), O.new_cache(4096, 1)
        O.append(1, kc, vc, 0, kn, v, O.rope_tables(0, 256))
        shas.append(np.stack([sha(kc[:256]), sha(vc[:256])]))
    e["rows_f32_sha"] = np.stack(shas)
    # flint_full (f32 cache of ctx rows) and flint_slide (f16 ring of 1024 rows, window 513)
    kc, vc = O.fl_new_cache(4096, 1), O.fl_new_cache(4096, 1)
    O.fl_kv_write(1, kc, vc, 0, x["fl_full_k"], x["fl_full_v"])
    e["flint_full"] = O.fl_attn_fd(1, kc, vc, x["fl_full_q"], 299, 0, x["fl_sinks"])
    kc, vc = O.fl_new_cache(1024, 0), O.fl_new_cache(1024, 0)
    O.fl_kv_write(0, kc, vc, 0, x["fl_slide_k"], x["fl_slide_v"])
    e["flint_slide"] = O.fl_attn_fd(0, kc, vc, x["fl_slide_q"], 1499, 513, x["fl_sinks"])
    return e


def generator_pins():
    """The first 4 values of a few streams, to pin normals() itself."""
    return np.stack([normals(s, (4,)) for s in (0, 1, 101, 2 ** 20)])


def main():
    import sys
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
    x = inputs()
    e = expected(x)
    np.savez_compressed(PATH, gen_pins=generator_pins(), pf_sel=PF_SEL, **e)
    print(f"wrote {PATH}: {os.path.getsize(PATH)} bytes, {len(e) + 2} arrays")


if __name__ == "__main__":
    main()
