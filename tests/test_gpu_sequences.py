"""Seeded random call sequences on one store, as an engine issues them: appends of ragged sizes, rollbacks of rejected
drafts (set_len), fused append + decode steps of 1-4 tokens, decodes and prefill blocks of random sizes and windows,
interleaved. The oracle keeps its own copy of the cache, fed the same appends (orc_append), and every attention
output is compared with the oracle function of the reference kernel that call takes, at that kernel's bar; at the
end the store's rows equal the oracle's bit for bit.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_attn_close, kv_inputs, prefill_reference, q_inputs

pytestmark = pytest.mark.gpu

F16, F32 = 0, 1
CTX = 4096


@pytest.fixture(scope="module")
def mk(torch_gpu):
    import mechta_amd
    mechta_amd.lib()
    return mechta_amd


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def decode_reference(fmt, kc, vc, q, n, start):
    """(reference, atol, rtol) of a decode: f16 one token or a window: attn_fd (f32-class); f16 2-4 tokens: attn_dmx;
    f32 store: attn_fd at 1e-5 (quad.rs:119-131, engine.rs:983-996)."""
    if fmt == F32:
        return O.attn_fd(F32, kc, vc, q, n, start=start), 1e-5, 1e-5
    if q.shape[0] == 1 or start > 0:
        return O.attn_fd(F16, kc, vc, q, n, start=start), 2e-3, 1e-3
    return O.attn_dmx(kc, vc, q, n), 2e-3, 1e-3


@pytest.mark.parametrize("fmt", [F16, F32])
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_call_sequence(torch_gpu, mk, fmt, seed):
    torch = torch_gpu
    r = np.random.default_rng(1000 * seed + fmt)
    kc, vc = O.new_cache(CTX, fmt), O.new_cache(CTX, fmt)
    length, step = 0, 0
    with mk.KvStore(1, CTX, fmt) as st:
        def append(m):
            nonlocal length, step
            kn, v = kv_inputs(10 * seed + step, m)
            tab = O.rope_tables(length, m)
            st.append(0, length, dev(torch, kn), dev(torch, v), dev(torch, tab))
            O.append(fmt, kc, vc, length, kn, v, tab)
            length += m

        append(int(r.integers(100, 350)))  # appends of at most MKV_PREFILL_MAX (512) rows each
        append(int(r.integers(100, 350)))
        for step in range(1, 40):
            op = r.choice(["append", "rollback", "verify", "decode", "prefill"], p=[0.2, 0.15, 0.3, 0.2, 0.15])
            if length > CTX - 600:
                op = "rollback_far"
            what = f"fmt={fmt} seed={seed} step {step}: {op} at length {length}"
            print(what, flush=True)
            if op == "append":
                append(int(r.integers(1, 49)))
            elif op == "rollback":
                length -= int(r.integers(1, 4))
                st.set_len(length)
            elif op == "rollback_far":
                length -= int(r.integers(300, 500))
                st.set_len(length)
            elif op == "verify":  # fused append of nt rows at the length, then the decode of those nt tokens
                nt = int(r.integers(1, 5))
                kn, v = kv_inputs(10 * seed + step, nt)
                tab = O.rope_tables(length, nt)
                q = q_inputs(20 * seed + step, nt)
                start = int(r.integers(0, length)) if r.random() < 0.2 else 0
                out = st.append_decode(0, length + 1, dev(torch, kn), dev(torch, v), dev(torch, tab), dev(torch, q),
                                       start=start).cpu().numpy()
                O.append(fmt, kc, vc, length, kn, v, tab)
                ref, atol, rtol = decode_reference(fmt, kc, vc, q, length + 1, start)
                length += nt
                assert_attn_close(out, ref, atol=atol, rtol=rtol, what=what)
            elif op == "decode":
                nt = int(r.integers(1, 5))
                n = int(r.integers(max(1, length - 400), length - nt + 2))
                start = int(r.integers(0, n)) if r.random() < 0.3 else 0
                q = q_inputs(30 * seed + step, nt)
                out = st.decode(0, dev(torch, q), n, start=start).cpu().numpy()
                ref, atol, rtol = decode_reference(fmt, kc, vc, q, n, start)
                assert_attn_close(out, ref, atol=atol, rtol=rtol, what=what)
            else:  # a prefill block ending at the length
                T = int(r.choice([1, 3, 8, 17, 32, 63, 64, 65, 100, 130]))
                T = min(T, length)
                n = length - T + 1
                start = int(r.integers(0, n)) if r.random() < 0.3 else 0
                q = q_inputs(40 * seed + step, T) / 4
                out = st.prefill(0, dev(torch, q), n, start=start).cpu().numpy()
                ref, atol, rtol = prefill_reference(fmt, kc, vc, q, n, start=start)
                assert_attn_close(out, ref, atol=atol, rtol=rtol, what=what)
        rows_k = st.read_rows(0, 0, 0, length).cpu().numpy()
        rows_v = st.read_rows(0, 1, 0, length).cpu().numpy()
    if fmt == F16:
        rows_k, rows_v = rows_k.view(np.uint16), rows_v.view(np.uint16)
    assert np.array_equal(rows_k.reshape(length, -1), kc[:length].reshape(length, -1)), "K rows differ from the oracle"
    assert np.array_equal(rows_v.reshape(length, -1), vc[:length].reshape(length, -1)), "V rows differ from the oracle"
