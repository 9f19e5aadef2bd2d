"""CPU checks of the boundary: the C-ABI library loads and exports every symbol include/mechta_kv.h declares, and
the host-side code needs no GPU (rope_table, error reporting). No compute call is made here."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import mechta_amd as mk
from oracle import oracle as O
from tests.helpers import fnv1a64, write_root_py

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mechta_kv.h")


def declared_symbols():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mkv_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = mk.lib()
    names = declared_symbols()
    assert len(names) >= 18
    for name in names:
        assert hasattr(lib, name), f"{name} missing from {mk.LIB_PATH}"
    assert sorted(mk.SYMBOLS) == names
    out = subprocess.run(["nm", "-D", "--defined-only", mk.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (mkv_\w+)", out))
    assert set(names) <= exported


def test_header_compiles_as_c():
    r = subprocess.run(["gcc", "-fsyntax-only", "-Wall", "-Werror", "-x", "c", HEADER], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("pos", [0, 1, 7, 4095, 65536, 262143])
def test_host_rope_table_matches_oracle(pos):
    """The library's host rope_table and the oracle's are the same f32 recurrence on the same libm: bit-equal."""
    got = np.array(mk.rope_table(pos), np.float32)
    assert np.array_equal(got, O.rope_table(pos))


def test_errors_without_gpu():
    lib = mk.lib()
    h = ctypes.c_void_p()
    assert lib.mkv_create(ctypes.byref(h), 1, 5000, mk.F16, None) == mk.E_CTX
    assert b"multiple of 1024" in lib.mkv_last_error()
    assert lib.mkv_create(ctypes.byref(h), 1, 4096, 7, None) == mk.E_ARG
    assert lib.mkv_create(None, 1, 4096, mk.F16, None) == mk.E_ARG
    assert lib.mkv_decode(None, 0, None, 1, 1, 0, 1.0, None, None) == mk.E_ARG
    assert lib.mkv_snapshot_bytes(None, 10) == 0


def test_store_bytes_known_answer():
    """The reference's one known-answer size (memcheck.rs:110-111): 22 buffers (K and V of 10 attention layers + the
    MTP layer) of 65,536 f32 positions = 2,952,790,016 bytes. The planes of a store of those 11 layers are exactly
    that (the blocked layout has no padding at a multiple of 1024 positions); the store allocates the stated
    overhead on top: 64 KiB of slack, the decode partials (2 x 32 rows x 256 splits x 1,040 B) and the prefill
    partials (2 x 4,096 (token, split) pairs x 8 heads x 1,040 B)."""
    assert 2 * 11 * mk.buffer_bytes(65536, mk.F32) == 2_952_790_016
    assert mk.buffer_bytes(65536, mk.F16) * 2 == mk.buffer_bytes(65536, mk.F32)
    overhead = 65536 + 2 * 32 * 256 * 1040 + 2 * 4096 * 8 * 1040
    assert mk.store_bytes(11, 65536, mk.F32) == 2_952_790_016 + overhead
    # f16 halves the planes only; fewer decode splits below 16,256 positions
    assert mk.store_bytes(11, 65536, mk.F16) == 2_952_790_016 // 2 + overhead
    assert mk.store_bytes(1, 4096, mk.F16) == 4096 * 512 * 2 * 2 + 65536 + 2 * 32 * 66 * 1040 + 2 * 4096 * 8 * 1040
    # cfg4: 10 f16 layers at 262,144 positions, 5.37 GB of planes
    assert mk.store_bytes(10, 262144, mk.F16) - overhead == 5_368_709_120
    # what mkv_create refuses has no size
    assert mk.store_bytes(1, 5000, mk.F16) == 0 and mk.store_bytes(1, 4096, 3) == 0 and mk.store_bytes(0, 4096, 0) == 0


# ---- root files: key and container parsing (host code only) ----

def test_fnv1a64_published_vectors():
    # FNV-1a 64 test vectors published with the algorithm (Fowler/Noll/Vo test suite)
    assert fnv1a64(b"") == 0xCBF29CE484222325
    assert fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert fnv1a64(b"foobar") == 0x85944171F73967E8


def test_root_key_is_fnv1a_of_token_bytes():
    r = np.random.default_rng(5)
    for n in (0, 1, 7, 2048):
        tok = r.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        assert mk.root_key(tok) == fnv1a64(tok.astype("<u4").tobytes())
    assert mk.root_key(np.frombuffer(b"foob", "<u4")) == fnv1a64(b"foob")


def test_root_info_reads_the_reference_layout(tmp_path):
    r = np.random.default_rng(6)
    p, nk = 5, 3
    tok = np.arange(100, 100 + p, dtype=np.uint32)
    ssm = [r.standard_normal(7).astype(np.float32), r.standard_normal(0).astype(np.float32)]
    conv = [r.standard_normal(3).astype(np.float32), r.standard_normal(11).astype(np.float32)]
    kv = [(r.integers(0, 2**32, p * 256, dtype=np.uint64).astype(np.uint32),
           r.integers(0, 2**32, p * 256, dtype=np.uint64).astype(np.uint32)) for _ in range(nk)]
    f = tmp_path / "root.bin"
    write_root_py(f, p, tok, ssm, conv, kv)
    info = mk.root_info(f)
    assert info == dict(p=p, ns=2, nk=nk, kv_words=p * 256, ssm_words=[7, 0], conv_words=[3, 11])
    b = f.read_bytes()
    for cut in (3, 14, 20, 38, len(b) - 4 * p * 256 - 1, len(b) - 1):  # truncated anywhere: refused
        g = tmp_path / f"cut{cut}.bin"
        g.write_bytes(b[:cut])
        with pytest.raises(mk.MkvError) as e:
            mk.root_info(g)
        assert e.value.code == mk.E_IO
    g = tmp_path / "bad.bin"
    g.write_bytes(b"MECHTA-ROOT-2\n" + b[14:])
    with pytest.raises(mk.MkvError) as e:
        mk.root_info(g)
    assert e.value.code == mk.E_IO
    with pytest.raises(mk.MkvError) as e:
        mk.root_info(tmp_path / "missing.bin")
    assert e.value.code == mk.E_IO


def test_build_keeps_packed_fp32_off_for_every_source():
    """Every HIP source is compiled with the packed-FP32 feature off (its v_pk_* f32 forms are not used on this
    hardware), and no per-file flag set turns it back on."""
    from mechta_amd import build as b
    flags = b.FLAGS
    i = flags.index("-target-feature")
    assert flags[i - 1] == "-Xclang" and flags[i + 1] == "-Xclang" and flags[i + 2] == "-packed-fp32-ops"
    for src, extra in b.EXTRA.items():
        assert src in b.SOURCES, src
        assert not any("packed-fp32" in x for x in extra), (src, extra)


def test_build_refuses_unreviewed_extra_flags(monkeypatch):
    """MKV_EXTRA_FLAGS reaches hipcc only in a development build (MKV_DEV_BUILD=1), and never when it names the
    packed-FP32 feature: a shipped library cannot silently turn packed FP32 back on."""
    from mechta_amd import build as b
    monkeypatch.delenv("MKV_DEV_BUILD", raising=False)
    monkeypatch.delenv("MKV_EXTRA_FLAGS", raising=False)
    assert b._extra_flags() == []
    monkeypatch.setenv("MKV_EXTRA_FLAGS", "-DFL_FUSE_NCH=4")
    with pytest.raises(RuntimeError):
        b._extra_flags()
    monkeypatch.setenv("MKV_DEV_BUILD", "1")
    assert b._extra_flags() == ["-DFL_FUSE_NCH=4"]
    monkeypatch.setenv("MKV_EXTRA_FLAGS", "-Xclang -target-feature -Xclang +packed-fp32-ops")
    with pytest.raises(RuntimeError):
        b._extra_flags()
    with pytest.raises(RuntimeError):  # the compile step itself refuses, before hipcc runs
        b._compile("kv_append.hip", False)


def test_root_path_matches_the_reference_naming(tmp_path):
    """root-<fmt>-<model key>-<token key>.bin, the model key FNV-1a over the path's bytes each widened to a u32 token
    (root_file / root_key, session.rs:62-73), checked against an independent FNV-1a."""
    model = "/models/Qwen3.6-35B-A3B-UD-Q4_K_S.gguf"
    toks = [151644, 8948, 198, 2610, 525]
    mkey = fnv1a64(np.array(list(model.encode()), np.uint32).tobytes())
    tkey = fnv1a64(np.array(toks, np.uint32).tobytes())
    assert mk.root_path(str(tmp_path), mk.F16, model, toks) == f"{tmp_path}/root-f16-{mkey:016x}-{tkey:016x}.bin"
    assert mk.root_path("/c", mk.F32, model, []).startswith(f"/c/root-f32-{mkey:016x}-{fnv1a64(b''):016x}")
    buf = ctypes.create_string_buffer(10)
    t = np.array(toks, np.uint32)
    assert mk.lib().mkv_root_path(buf, 10, b"/c", mk.F16, model.encode(), t.ctypes.data_as(ctypes.c_void_p),
                                  t.size) == mk.E_SIZE
    assert mk.lib().mkv_root_path(buf, 10, b"/c", 7, model.encode(), None, 0) == mk.E_ARG
    assert mk.ROOT_MIN == 2048


def test_root_prune_keeps_the_most_recent(tmp_path):
    """prune_roots (session.rs:75-84): only root-<fmt>-*.bin files count; the `keep` newest stay, at least one;
    mkv_root_touch makes a file the newest."""
    for i in range(8):
        f = tmp_path / f"root-f16-m-{i:02d}.bin"
        f.write_bytes(b"x")
        os.utime(f, (1000 + i, 1000 + i))
    for name in ("root-f32-m-00.bin", "root-f16-m-99.bin.tmp", "other.bin"):
        (tmp_path / name).write_bytes(b"y")
        os.utime(tmp_path / name, (1, 1))
    mk.root_touch(str(tmp_path / "root-f16-m-00.bin"))  # oldest becomes newest
    assert mk.root_prune(str(tmp_path), mk.F16, 6) == 2
    left = sorted(p.name for p in tmp_path.iterdir())
    assert left == ["other.bin", "root-f16-m-00.bin", "root-f16-m-03.bin", "root-f16-m-04.bin", "root-f16-m-05.bin",
                    "root-f16-m-06.bin", "root-f16-m-07.bin", "root-f16-m-99.bin.tmp", "root-f32-m-00.bin"]
    assert mk.root_prune(str(tmp_path), mk.F16, 0) == 5  # keep at least one: the newest
    assert (tmp_path / "root-f16-m-00.bin").exists()
    assert mk.root_prune(str(tmp_path / "missing"), mk.F16, 6) == 0
    with pytest.raises(mk.MkvError) as e:
        mk.root_touch(str(tmp_path / "missing.bin"))
    assert e.value.code == mk.E_IO
