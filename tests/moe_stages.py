"""Stage-by-stage parity of one MoE layer call (purhie_moe_ffn), shared by the GPU tests.

After a call, the layer's own intermediate results are read back from its workspace (purhie_moe_debug_regions,
include/moe_layer.h) and each stage is checked on the GPU's own inputs to it, at the path's bounds: the routed ids
and the combine bit for bit (the routing weights within 2e-6), every down projection within 1e-5 sum |w x|
(tests/matvec_verify.cpp:8,142). The whole layer against the oracle's own composition is only a reading (2e-3 of the row maximum): there the fp32
order of the gate / up sums can move one re-quantized SwiGLU value by a step, and the stages cannot.
"""
import numpy as np

from tests import parity

KQ = (12, 13, 14, 23)


def q8_host(ws, off, k, kq):
    """rows of n values of the qmatvec_q8 of k values at byte offset off of the host copy ws (qmatvec_q8_bind's
    layout: q0, qK, d0, dK, bsK, s0 in 16-byte aligned sections), as the oracle's activation dicts"""
    a16 = lambda n: (n + 15) // 16 * 16
    q0o, qKo = off, off + a16(k)
    d0o = off + 2 * a16(k)
    dKo = d0o + a16(k // 32 * 4)
    bsKo = dKo + a16(k // 256 * 4)

    def row(i, n):
        b = i * n
        if kq:
            return dict(q=ws[qKo + b:qKo + b + n].view(np.int8),
                        d=ws[dKo + b // 256 * 4:dKo + (b + n) // 256 * 4].view(np.float32),
                        bs=ws[bsKo + b // 16 * 4:bsKo + (b + n) // 16 * 4].view(np.int32))
        return dict(q=ws[q0o + b:q0o + b + n].view(np.int8),
                    d=ws[d0o + b // 32 * 4:d0o + (b + n) // 32 * 4].view(np.float32))
    return row


def check(M, oracle, w, x, logits, out, ws, down_w, t_d, NU, sdown_w=None, t_sd=None, FS=0, rows=None):
    """the routed ids bit for bit (weights within 2e-6) against the oracle's router on the same logits; every
    slot's down projection of the activation the GPU formed (its quantized SwiGLU, or the oracle's quantization of the GPU's gate and up outputs
    where the down launch forms it in-kernel) within 1e-5 sum |w x|, and the quantized SwiGLU bit for bit where both
    exist; the shared expert's down the same way; the combine of the GPU's down outputs, weights, shared output and
    gate bit for bit. rows: the tokens whose down projections are checked (default all)"""
    T, E, FE = x.shape[0], w.n_embd, w.n_ff_exp
    r = M.regions(w, T)
    ns = r.ns
    f32 = lambda off, n: ws[off:off + 4 * n].view(np.float32)
    ids = ws[r.ids:r.ids + 4 * T * ns].view(np.int32).reshape(T, ns)
    wts = f32(r.wts, T * NU).reshape(T, NU)
    oid, ow = oracle.moe_router(logits, NU)
    assert np.array_equal(ids[:, :NU], oid), "routed ids"
    # (the softmax's sum runs in a wave-reduction order and uses the device's expf: the weights agree to a few
    # ulp, as tests/test_gpu_moe.py's router test bounds them; every later stage is fed the GPU's own weights)
    assert np.allclose(wts, ow, rtol=2e-6, atol=1e-8), "routing weights"
    kq_d = t_d in KQ
    down = f32(r.down, T * ns * E).reshape(T * ns, E)
    qx = q8_host(ws, r.qx, r.qx_k, kq_d)
    if r.gu_written:
        g = f32(r.g, T * ns * FE).reshape(T * ns, FE)
        u = f32(r.u, T * ns * FE).reshape(T * ns, FE)
    for t in (range(T) if rows is None else rows):
        for j in range(ns):
            i = t * ns + j
            if r.gu_written:
                act = oracle.quantize_act(oracle.swiglu(g[i], u[i]), kq_d)
                if r.act_written:
                    got = qx(i, FE)
                    assert np.array_equal(got["q"], act["q"]) and \
                        np.array_equal(got["d"].view(np.uint32), act["d"].view(np.uint32)), f"SwiGLU of row {i}"
            else:
                act = qx(i, FE)
            e = ids[t, j]
            Wd = sdown_w if e < 0 else down_w[e * E:(e + 1) * E]
            want, _, mag = oracle.matvec(t_d, Wd, E, FE, act, False)
            parity.check("MoE layer: down of the GPU's activation", down[i], want, mag)
    shared, sg = None, None
    if sdown_w is not None and not r.slot:
        kq_s = t_sd in KQ
        shared = f32(r.shout, T * E).reshape(T, E)
        qs = q8_host(ws, r.qs, r.qs_k, kq_s)
        for t in (range(T) if rows is None else rows):
            want, _, mag = oracle.matvec(t_sd, sdown_w, E, FS, qs(t, FS), False)
            parity.check("MoE layer: shared down of the GPU's activation", shared[t], want, mag)
    elif sdown_w is not None:
        shared = down.reshape(T, ns, E)[:, NU]
    if r.sg >= 0:
        sg = f32(r.sg, T)
    comb = oracle.moe_combine(down.reshape(T, ns, E)[:, :NU], wts, shared, sg)
    assert np.array_equal(out.view(np.uint32), comb.view(np.uint32)), "combine of the GPU's stages"
    return r
