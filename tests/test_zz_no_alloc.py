"""mkv_append_decode_noalloc (the allocation-free verify step, its partials in the library's per-GPU scratch array)
against mkv_append_decode (the handle's workspace), through the C ABI: two calls in a row on each store format, the
second with a smaller input (fewer tokens, a shorter context: fewer splits), outputs and appended rows bit-identical
(the same kernels run on the same inputs), and the first also within the task tolerance of the oracle."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_attn_close, gate_inputs, kv_inputs, q_inputs

pytestmark = pytest.mark.gpu

F16, F32 = 0, 1


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("fmt", [F16, F32])
def test_noalloc_verify_equals_the_workspace_entry(torch_gpu, fmt):
    import mechta_amd as mk
    torch = torch_gpu
    lib = mk.lib()
    ctx = 20480
    steps = [(19000, 4, 0), (1500, 2, 0)]  # (n, ntok, start): the second smaller
    npos = 19000 + 3
    kn, v = kv_inputs(90 + fmt, npos)
    tab = O.rope_tables(0, npos)
    with mk.KvStore(1, ctx, fmt) as a, mk.KvStore(1, ctx, fmt) as b:
        for st in (a, b):
            for p in range(0, 19000 - 1, 512):
                m = min(512, 19000 - 1 - p)
                st.append(0, p, _dev(torch, kn[p:p + m]), _dev(torch, v[p:p + m]), _dev(torch, tab[p:p + m]))
        for i, (n, ntok, start) in enumerate(steps):
            print(f"noalloc fmt={fmt} call {i}: n={n} ntok={ntok}", flush=True)
            a.set_len(n - 1)
            b.set_len(n - 1)
            q = _dev(torch, q_inputs(95 + i, ntok))
            g = _dev(torch, gate_inputs(97 + i, ntok))
            ins = [_dev(torch, x[n - 1:n - 1 + ntok]) for x in (kn, v, tab)]
            oa = torch.full((ntok, 16, 256), float("nan"), device="cuda")
            ob = torch.full((ntok, 16, 256), float("nan"), device="cuda")
            rc = lib.mkv_append_decode(a._h, 0, n, ntok, *[_p(x) for x in ins], _p(q), start, 1.0 / 16, _p(oa), _p(g))
            assert rc == 0, lib.mkv_last_error()
            rc = lib.mkv_append_decode_noalloc(b._h, 0, n, ntok, *[_p(x) for x in ins], _p(q), start, 1.0 / 16,
                                               _p(ob), _p(g))
            assert rc == 0, lib.mkv_last_error()
            torch.cuda.synchronize()
            assert torch.isfinite(ob).all()
            assert torch.equal(oa, ob), f"call {i}: outputs differ"
            for w in (mk.K, mk.V):
                assert torch.equal(a.read_rows(0, w, n - 1, n - 1 + ntok), b.read_rows(0, w, n - 1, n - 1 + ntok))
            if i == 0:
                kc, vc = O.new_cache(ctx, fmt), O.new_cache(ctx, fmt)
                O.append(fmt, kc, vc, 0, kn[:n - 1 + ntok], v[:n - 1 + ntok], tab[:n - 1 + ntok])
                qn = q.cpu().numpy()
                att = O.attn_dmx(kc, vc, qn, n) if fmt == F16 else O.attn_fd(F32, kc, vc, qn, n)
                ref = O.gate(att, g.cpu().numpy()).reshape(ntok, 16, 256)
                tol = {} if fmt == F16 else {"atol": 1e-5, "rtol": 1e-5}
                assert_attn_close(ob.cpu().numpy(), ref, what="noalloc vs oracle", **tol)


def test_noalloc_records_no_trace_and_replays_under_capture(torch_gpu):
    """The no-allocation call takes no trace events, even with the handle's trace on (taking them may create events
    and grows a host list), and it captures into a HIP graph (global capture mode, where an allocation would fail the
    capture) whose replays, with eager work of the same store in between, equal the eager call bit for bit."""
    import mechta_amd as mk
    torch = torch_gpu
    lib = mk.lib()
    n0, ntok = 3000, 4
    print("noalloc: trace and capture", flush=True)
    kn, v = kv_inputs(181, n0 + ntok)
    tab = O.rope_tables(0, n0 + ntok)
    q = _dev(torch, q_inputs(182, ntok))
    with mk.KvStore(1, 8192, F16) as st:
        for p in range(0, n0 - 1, 512):
            m = min(512, n0 - 1 - p)
            st.append(0, p, _dev(torch, kn[p:p + m]), _dev(torch, v[p:p + m]), _dev(torch, tab[p:p + m]))
        ins = [_dev(torch, x[n0 - 1:n0 - 1 + ntok]) for x in (kn, v, tab)]
        st.trace(True)
        out_e = torch.full((ntok, 16, 256), float("nan"), device="cuda")
        rc = lib.mkv_append_decode_noalloc(st.handle, 0, n0, ntok, *[_p(x) for x in ins], _p(q), 0, 1.0 / 16,
                                           _p(out_e), None)
        assert rc == 0, lib.mkv_last_error()
        spans = st.trace_read()
        assert spans["core"][1] == 0 and spans["merge"][1] == 0, spans
        assert torch.isfinite(out_e).all()
        st.set_len(n0 - 1)
        out_g = torch.empty((ntok, 16, 256), device="cuda")
        g = torch.cuda.CUDAGraph()
        base = torch.cuda.current_stream()
        with torch.cuda.graph(g):
            st.set_stream(torch.cuda.current_stream())
            rc = lib.mkv_append_decode_noalloc(st.handle, 0, n0, ntok, *[_p(x) for x in ins], _p(q), 0, 1.0 / 16,
                                               _p(out_g), None)
        st.set_stream(base)
        assert rc == 0, lib.mkv_last_error()
        st.trace(False)
        for r in range(3):
            out_g.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_g, out_e), f"replay {r} differs from the eager call"
            other = st.decode(0, q, n0 - 700)
            torch.cuda.synchronize()
            assert torch.isfinite(other).all()
