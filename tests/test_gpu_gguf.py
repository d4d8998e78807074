"""GGUF tensors staged into HBM (gguf_hbm_stage) and bound (gguf_bind_weight): the device copies equal the file's
bytes, the model then hands out device addresses inside the caller's buffer, unstaged tensors keep pointing into
the mapping, and a matvec on a bound Q4_K weight and a grouped-GEMM over a bound 3-D ROCmFP4 expert stack match
the oracle (bit for bit against the same launch on a torch copy of the bytes). A multi-chunk file exercises the
pinned ring."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import gguf as G
from purhie_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def Q():
    from purhie_amd import qmatvec
    qmatvec.lib()
    return qmatvec


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_stage_bind_and_matvec(Q, oracle, tmp_path):
    import torch
    N, K = 512, 2560
    Wq = oracle.quantize(12, synth.gaussian(71, N * K, 0, 0.02).reshape(N, K))
    E, F, H = 4, 64, 256
    We = oracle.quantize(100, synth.gaussian(72, E * F * H, 0, 0.02).reshape(E * F, H))
    norm = synth.gaussian(73, K)
    p = tmp_path / "w.gguf"
    G.write(p, [("general.architecture", G.STRING, "qwen3")],
            [("blk.0.ffn_gate.weight", 12, (K, N), Wq.tobytes()), ("blk.0.attn_norm.weight", 0, (K,), norm.tobytes()),
             ("blk.0.ffn_up_exps.weight", 100, (H, F, E), We.tobytes())])
    with G.Model(p) as m:
        keep = np.array([1, 0, 1], np.uint8)
        need = m.hbm_bytes(keep)
        buf = torch.zeros(need + 4096, dtype=torch.uint8, device="cuda")
        src_norm = m.tensor("blk.0.attn_norm.weight")[0]
        rc, got_need = m.hbm_stage(buf, keep)
        assert rc == 0 and got_need == need
        base = buf.data_ptr()
        rc, w = m.bind_weight("blk.0.ffn_gate.weight")
        assert rc == 0 and (w.type, w.N, w.K) == (12, N, K) and base <= w.data < base + need
        off = w.data - base
        dW = buf[off:off + N * w.row_bytes]
        assert np.array_equal(host(dW), Wq.reshape(-1).view(np.uint8))
        assert m.tensor("blk.0.attn_norm.weight")[0] == src_norm  # not kept: still the mapping
        rc, we = m.bind_weight("blk.0.ffn_up_exps.weight")
        assert rc == 0 and (we.N, we.K) == (E * F, H)
        eoff = we.data - base
        assert eoff % 256 == 0 and np.array_equal(host(buf[eoff:eoff + E * F * we.row_bytes]),
                                                   We.reshape(-1).view(np.uint8))
        # a matvec on the bound (device-resident) weight
        x = synth.gaussian(74, K)
        q = Q.Q8(K)
        Q.quantize(torch.from_numpy(x).cuda(), K, q)
        y = torch.zeros(N, dtype=torch.float32, device="cuda")
        Q.launch_q8(12, dW, q, y, N, K)
        y2 = torch.zeros(N, dtype=torch.float32, device="cuda")
        Q.launch_q8(12, torch.from_numpy(Wq.reshape(-1).view(np.uint8).copy()).cuda(), q, y2, N, K)
        got = host(y)
        assert np.array_equal(got.view(np.uint32), host(y2).view(np.uint32))
        want, _, mag = oracle.matvec(12, Wq, N, K, oracle.quantize_act(x, True))
        assert np.all(np.abs(got - want) <= 1e-5 * mag)


def test_multi_chunk_stage(Q, tmp_path):
    """a file larger than the pinned ring (3 x 64 MiB): every byte arrives, tensors at 256-byte offsets"""
    import time

    import torch
    rng = np.random.default_rng(5)
    sizes = [150 << 20, 37 << 20, 3 * 34 + 0, 90 << 20]  # Q8_0 tensors of these many bytes (34-byte blocks)
    tensors = []
    for i, s in enumerate(sizes):
        nb = max(1, s // 34)
        tensors.append((f"t{i}", 8, (32 * nb,), rng.integers(0, 256, nb * 34, dtype=np.uint8).tobytes()))
    p = tmp_path / "big.gguf"
    G.write(p, [], tensors)
    with G.Model(p) as m:
        need = m.hbm_bytes()
        buf = torch.empty(need, dtype=torch.uint8, device="cuda")
        t0 = time.perf_counter()
        rc, _ = m.hbm_stage(buf)
        dt = time.perf_counter() - t0
        assert rc == 0
        print(f"staged {need / 1e6:.0f} MB in {dt * 1e3:.1f} ms ({need / dt / 1e9:.1f} GB/s)", flush=True)
        base = buf.data_ptr()
        for name, _, _, data in tensors:
            ptr, n = m.tensor(name)
            assert n == len(data) and (ptr - base) % 256 == 0
            got = host(buf[ptr - base:ptr - base + n])
            assert np.array_equal(got, np.frombuffer(data, np.uint8)), name
        small = torch.empty(need - 1, dtype=torch.uint8, device="cuda")
        assert m.L.gguf_hbm_stage(m.h, C.c_void_p(small.data_ptr()), small.numel(), None, None) == -1
