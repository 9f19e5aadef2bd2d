"""The path under HIP graph capture. The reference records its commands once and replays them every step
(engine.rs:571-597; only uniforms change); the MI355X equivalent is a captured graph. A verify step
(mkv_append_decode: fused append + decode + merge), its gated f16 output (mkv_decode_g16) and a prefill are captured through the C ABI on torch's capture
stream and replayed several times, with eager work of the same store in between; every replay must equal the eager
call of the same step bit for bit (a captured step re-appends its rows at the same positions, so replays are
idempotent). The calls make no allocation, host synchronization or memset once the store exists: the graph is
captured before any eager attention call of the store.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import gate_inputs, kv_inputs, q_inputs

pytestmark = pytest.mark.gpu

F16, F32 = 0, 1


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("fmt", [F16, F32])
def test_captured_verify_and_prefill_replay_bit_identical(torch_gpu, fmt):
    import mechta_amd as mk
    torch = torch_gpu
    print(f"graph capture fmt={fmt}", flush=True)
    n0, ntok, T, Ts = 3000, 4, 64, 24
    kn, v = kv_inputs(71, n0 + T)
    tab = O.rope_tables(0, n0 + T)
    q4, q64, q24 = _dev(torch, q_inputs(72, ntok)), _dev(torch, q_inputs(73, T)), _dev(torch, q_inputs(74, Ts))
    qf = _dev(torch, gate_inputs(75, ntok))
    with mk.KvStore(1, 8192, fmt) as st:
        for p in range(0, n0 - 1, 512):
            m = min(512, n0 - 1 - p)
            st.append(0, p, _dev(torch, kn[p:p + m]), _dev(torch, v[p:p + m]), _dev(torch, tab[p:p + m]))
        step_in = [_dev(torch, a[n0 - 1:n0 - 1 + ntok]) for a in (kn, v, tab)]
        torch.cuda.synchronize()
        # captured first, on a store that has run no attention yet: nothing is allocated or grown by the calls
        out_g = torch.empty((ntok, 16, 256), device="cuda")
        pf_g = torch.empty((T, 16, 256), device="cuda")
        ps_g = torch.empty((Ts, 16, 256), device="cuda")
        h_g = torch.empty((ntok, 16, 256), dtype=torch.float16, device="cuda")
        g = torch.cuda.CUDAGraph()
        base_stream = torch.cuda.current_stream()
        with torch.cuda.graph(g):
            st.set_stream(torch.cuda.current_stream())
            st.append_decode(0, n0, *step_in, q4, out=out_g)
            st.decode(0, q4, n0, gate_src=qf, f16_out=True, out=h_g)  # the gated f16 output (attn_gate16)
            st.prefill(0, q64, n0 + ntok - T, out=pf_g)   # the last T positions as a prefill block
            st.prefill(0, q24, n0 + ntok - Ts, out=ps_g)  # a small block (f32-class on the f16 store)
        st.set_stream(base_stream)
        st.set_len(n0 - 1)
        out_e = st.append_decode(0, n0, *step_in, q4).clone()
        h_e = st.decode(0, q4, n0, gate_src=qf, f16_out=True).clone()
        pf_e = st.prefill(0, q64, n0 + ntok - T).clone()
        ps_e = st.prefill(0, q24, n0 + ntok - Ts).clone()
        torch.cuda.synchronize()
        for r in range(4):
            for t in (out_g, pf_g, ps_g, h_g):
                t.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_g, out_e), f"replay {r}: verify output differs from the eager call"
            assert torch.equal(h_g, h_e), f"replay {r}: gated f16 output differs from the eager call"
            assert torch.equal(pf_g, pf_e), f"replay {r}: prefill output differs from the eager call"
            assert torch.equal(ps_g, ps_e), f"replay {r}: small prefill output differs from the eager call"
            # eager work of the same store between replays: a decode at another length
            other = st.decode(0, q4, n0 - 500)
            torch.cuda.synchronize()
            assert torch.isfinite(other).all()
