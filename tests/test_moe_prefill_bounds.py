"""CPU replay of every address the MoE prefill launches form, on the benchmark's own 512-token routing.

The five launches of config 4's prefill (bench.py bench_moe): k_moe_router, k_moe_group, the expert-tiled gate / up
GEMM with the SwiGLU epilogue (k_gemm_split<100, 64, 256, MoE, PD 4, SWP>), the down GEMM (k_gemm_split<100, 64,
256, MoE, PD 4>) and k_moe_combine. Each test restates one kernel's index arithmetic (moe.hip, moe_dev.h,
gemm_split.hip) over its whole grid, every (workgroup, thread) at once in numpy, and asserts that each global
and LDS access lies inside the buffer the launch binds it to, with the sizes bench.py allocates. The routing comes
from the C oracle's router on the benchmark's seeded logits (purhie_amd/synth.py) and its grouping: the GPU's
grouping differs only in the order of the entries inside an expert's run, and every address below depends on an
entry only through its own in-range row numbers, so the bounds hold for any such order.

No GPU is used. Reference: src/gpu_ops.hip:185-330 (router, group, combine) and src/matvec_q.hip:2948-2962 (the
expert-tiled GEMM) define what these kernels compute; the layouts checked here are this library's own.
"""
import numpy as np
import pytest

from oracle import oracle as O
from purhie_amd import synth

T, E, NU, H, F = 512, 128, 8, 2048, 768
N_ENT = T * NU
TILE = 64                    # qmatvec_id_batch_tile for the split GEMM's MoE tiles
ROWS, TT = 256, 64           # split GEMM MoE tile: weight rows, token entries
PD = 4                       # MoE prefetch distance: stages past the end reload the last one
BB = 18                      # ROCmFP4 block bytes
LOGIT_SEED = 0x5EED2104      # bench.py's prefill router logits


def row_size(K):
    return K // 32 * BB


def sp_at(r, ch):
    """gemm_split.hip's LDS place (bytes) of 16-byte chunk ch of a stage's row r"""
    return ((r >> 4) << 10) + (ch << 8) + ((r & 15) << 4)


def q8_sections(max_k):
    """byte sizes of qmatvec_q8's sections (qmatvec_q8_bind: q0, qK, d0, dK, bsK, s0)"""
    return dict(q0=max_k, qK=max_k, d0=max_k // 32 * 4, dK=max_k // 256 * 4, bsK=max_k // 16 * 4, s0=max_k // 32 * 4)


def inside(what, off, width, size):
    """every access [off, off + width) inside [0, size)"""
    off = np.asarray(off, dtype=np.int64)
    lo, hi = int(off.min()), int(off.max()) + width
    assert lo >= 0 and hi <= size, f"{what}: bytes [{lo}, {hi}) outside [0, {size})"


@pytest.fixture(scope="module")
def routing():
    logits = synth.gaussian(LOGIT_SEED, T * E).reshape(T, E)
    ids, wts = O.moe_router(logits, NU)
    g = O.moe_group(ids, E, TILE)
    mt = min(N_ENT, E + N_ENT // TILE)  # gpu_moe_max_tiles
    return dict(logits=logits, ids=ids, wts=wts, mt=mt, **g)


def test_router_addresses(routing):
    """k_moe_router: grid T, 256 threads, route_token_128 (n_expert <= 128)"""
    t = np.arange(T)[:, None]
    lane = np.arange(256)[None, :] & 63
    for col in (lane, lane + 64):
        live = np.broadcast_to(col < E, (T, 256))
        inside("logits", ((t * E + col) * 4)[live], 4, T * E * 4)
    ids = routing["ids"]
    # ids[r] = expert for rank r < n_used (ids_stride = n_used, no shared slot); wts[tid] for tid < n_used
    assert ids.min() >= 0 and ids.max() < E
    inside("ids", (t * NU + np.arange(NU)[None, :]) * 4, 4, N_ENT * 4)
    inside("wts", (t * NU + np.arange(NU)[None, :]) * 4, 4, N_ENT * 4)
    # LDS: wkey[4][128] (u64), part[4][128], read wkey[32 w + j .. + 1] for j < 32
    w = np.arange(4)[:, None]
    j = np.arange(0, 32, 2)[None, :]
    inside("wkey (LDS)", (w * 128 + 32 * w + j) * 8, 16, 4 * 128 * 8)


def test_group_addresses(routing):
    """k_moe_group: one workgroup of 1024 threads"""
    ids = routing["ids"].reshape(-1)
    i = np.arange(N_ENT)
    inside("ids", i * 4, 4, N_ENT * 4)
    assert ids.min() >= 0 and ids.max() < E  # cnt[e], slot[e]: LDS of MOE_MAX_EXPERTS = 1024 ints
    inside("cnt (LDS)", np.arange(1024) * 4, 4, 1024 * 4)
    nt, mt = routing["n_tiles"], routing["mt"]
    assert 0 < nt <= mt, (nt, mt)
    counts = np.bincount(ids, minlength=E)
    tiles_per = (counts + TILE - 1) // TILE
    to = np.concatenate([[0], np.cumsum(tiles_per)[:-1]])
    k = np.concatenate([to[e] + np.arange(tiles_per[e]) for e in range(E)])
    inside("tile_e / tile_start / tile_n", k * 4, 4, mt * 4)
    assert to[-1] + tiles_per[-1] == nt
    # tok_rows[p], pair_rows[p]: p = an atomic slot in expert e's run [eo, eo + c)
    eo = np.concatenate([[0], np.cumsum(counts)[:-1]])
    inside("tok_rows / pair_rows", (eo + counts - 1)[counts > 0] * 4, 4, N_ENT * 4)
    # the tiles cover each expert's run in order, tile_n <= TILE
    ts, tn = routing["tile_start"], routing["tile_n"]
    assert (tn >= 1).all() and (tn <= TILE).all() and (ts + tn <= N_ENT).all()


def split_gemm_replay(routing, N, K, swp, w_bytes, x_rows, y_or_h):
    """k_gemm_split<TY_FP4, 64, 256, MoE, PD 4, swp> over grid (N / 128 (swp) or N / 256, max_tiles)"""
    nt, mt = routing["n_tiles"], routing["mt"]
    te, ts, tn = routing["tile_e"], routing["tile_start"], routing["tile_n"]
    in_rows = routing["tok_rows"] if swp else routing["pair_rows"]
    out_rows = routing["pair_rows"]
    nb, rb = K // 32, row_size(K)
    assert nb % 2 == 0 and K % 64 == 0  # the host's K multiple (even stage count)
    gx = N // (ROWS // 2) if swp else (N + ROWS - 1) // ROWS
    tid = np.arange(256)
    lane, wave = tid & 63, tid >> 6
    sec = q8_sections(x_rows * K)
    assert routing["tile_e"].max() < E
    # workgroups with k >= *n_tiles return after reading n_tiles (offset 0); the rest read tile_*[k], k < nt <= mt
    inside("tile_e / tile_start / tile_n", np.arange(nt) * 4, 4, mt * 4)
    # the matrix bytes: every allocation ends on a 4-byte boundary, so a 4-aligned word holding a block's last
    # byte lies inside it
    assert w_bytes % 4 == 0
    VN, TPR = TT // 8, 32 // (TT // 8)
    xr, xp = tid // TPR, tid % TPR
    x0 = VN * xp
    lr = tid // (256 // ROWS)
    # LDS bytes of sW0 / sW1 (the SwiGLU epilogue's [32][129] floats share them) and of sX0 / sX1
    sw_bytes = 2 * (max(ROWS * 32, 2 * 32 * 129) if swp else ROWS * 32)
    sx_bytes = TT * 64
    stages = np.arange(nb + PD)  # the loop's issues: stages 0 .. nb - 1 + PD, clamped to nb - 1
    s_cl = np.minimum(stages, nb - 1)
    for k in range(nt):
        e, st, n = int(te[k]), int(ts[k]), int(tn[k])
        inside("in_rows / out_rows", (st + np.arange(n)) * 4, 4, N_ENT * 4)
        for bx in range(gx):
            n0 = bx * (ROWS // 2) if swp else bx * ROWS
            wr = n0 + (lr % (ROWS // 2) if swp else lr)
            wrow = (e * N + np.minimum(wr, N - 1)) * rb  # byte offset in W (or W2: the same size)
            b = wrow[:, None] + s_cl[None, :] * BB
            al = b - (b & 3)  # allocation bases are 256-aligned: the offset's low bits are the address's
            inside("W / W2 (five words from the aligned word)", al, 20, w_bytes)
            # the token rows: positions past the tile's entries repeat entry 0's row
            xrow = in_rows[st + np.where(xr < n, xr, 0)].astype(np.int64)
            assert xrow.max() < x_rows
            inside("xq = q0", (xrow * K + x0)[:, None] + 32 * s_cl[None, :], 8, sec["q0"])
            inside("dx = d0 (stages)", ((xrow * nb)[:, None] + s_cl[None, :]) * 4, 4, sec["d0"])
            inside("dx = d0 (the prologue's max)", (xrow * nb + nb - 1) * 4, 4, sec["d0"])
            # LDS: the weight row lr's four 16-byte chunks; the token row xr's chunks x0 / 8 ..
            inside("sW (LDS)", np.array([sp_at(lr, ch) for ch in range(4)]), 16, sw_bytes)
            inside("sX (LDS)", np.array([sp_at(xr, x0 // 8 + k) for k in range(VN // 8)]), 16, sx_bytes)
            # fragments: rows wr0 + 16 i + lane % 16, chunk lane / 16
            RT, CT = ROWS // 32, TT // 32
            wr0, wc0 = (wave >> 1) * RT * 16, (wave & 1) * CT * 16
            i = np.arange(RT)[None, :]
            inside("sW fragments (LDS)", sp_at(wr0[:, None] + 16 * i + (lane[:, None] & 15), lane[:, None] >> 4),
                   16, sw_bytes)
            jj = np.arange(CT)[None, :]
            tr = wc0[:, None] + 16 * jj + (lane[:, None] & 15)
            inside("sX fragments (LDS)", sp_at(tr, lane[:, None] >> 4), 16, sx_bytes)
            if swp:
                # up waves (2, 3) write u into their buffer of sW0 / sW1: [token][129] floats
                tl = 16 * np.arange(CT)[:, None] + (lane[None, :] & 15)
                u_idx = (tl[:, :, None] * 129 + 16 * np.arange(RT)[None, None, :] +
                         4 * (lane[None, :, None] >> 4))[..., None] + np.arange(4)
                inside("sU (LDS, in sW)", u_idx * 4, 4, sw_bytes)
                # gate waves (0, 1): quantized SwiGLU rows out_rows[tt] for tt < n
                for w_ in (0, 1):
                    tt = 16 * CT * (w_ & 1) + tl
                    st_ok = tt < n
                    if not st_ok.any():
                        continue
                    hrow = out_rows[st + tt[st_ok]].astype(np.int64)
                    hs = q8_sections(N_ENT * N)
                    ln = np.broadcast_to(lane[None, :], tt.shape)[st_ok]
                    for bq in range(RT // 2):
                        q0 = hrow * N + n0 + 32 * bq + 4 * (ln >> 4)
                        inside("hq (q0 bytes 0-3)", q0, 4, hs["q0"])
                        inside("hq (q0 bytes 16-19)", q0 + 16, 4, hs["q0"])
                        bi = hrow * (N // 32) + (n0 + 32 * bq) // 32
                        inside("hd / hs", bi * 4, 4, hs["d0"])
            else:
                for w_ in range(4):
                    tt = wc0[w_ * 64] + 16 * np.arange(CT)[:, None] + (lane[None, :] & 15)
                    ok = tt < n
                    if not ok.any():
                        continue
                    yrow = out_rows[st + tt[ok]].astype(np.int64) * N
                    ln = np.broadcast_to(lane[None, :], tt.shape)[ok]
                    nn = n0 + wr0[w_ * 64] + 16 * np.arange(RT)[:, None] + 4 * (ln[None, :] >> 4)
                    for r in range(4):
                        m = nn + r < N
                        inside("y", ((yrow[None, :] + nn + r)[m]) * 4, 4, y_or_h)


def test_gate_up_swiglu_gemm_addresses(routing):
    w_bytes = E * F * row_size(H)
    split_gemm_replay(routing, F, H, True, w_bytes, T, None)


def test_down_gemm_addresses(routing):
    w_bytes = E * H * row_size(F)
    split_gemm_replay(routing, H, F, False, w_bytes, N_ENT, N_ENT * H * 4)


def test_combine_addresses(routing):
    """k_moe_combine: grid (H / 256, T), 256 threads; no shared expert"""
    t = np.arange(T)[:, None]
    i = np.arange(H)[None, :]
    for j in range(NU):
        inside("down", ((t * NU * H + i) + j * H) * 4, 4, N_ENT * H * 4)
    inside("wts", (t * NU + np.arange(NU)[None, :]) * 4, 4, N_ENT * 4)
    inside("out", (t * H + i) * 4, 4, T * H * 4)


def test_replay_reaches_the_buffer_ends(routing):
    """the replay is tight: one word less of the weights, or one float less of the output, fails it"""
    with pytest.raises(AssertionError, match="W / W2"):
        split_gemm_replay(routing, F, H, True, E * F * row_size(H) - 4, T, None)
    with pytest.raises(AssertionError, match="y"):
        split_gemm_replay(routing, H, F, False, E * H * row_size(F), N_ENT, N_ENT * H * 4 - 4)
