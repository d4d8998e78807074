"""The GGUF reader (include/gguf_mmap.h) on files written by purhie_amd.gguf.write: every introspection result
against the values the files were written with, and against the reference's own reader (src/gguf_mmap.cpp,
compiled into oracle/_ref) call for call; the scalar getters' widening rules over every stored type; splits,
custom alignment, name truncation, bind_weight; and refusal of truncated or malformed files (where the
reference, which does not check extents, is not run)."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

from purhie_amd import gguf as G

GETTERS = ("u8", "i8", "u16", "i16", "u32", "i32", "f32", "u64", "i64", "f64")
SCALARS = [(G.U8, 200), (G.I8, -7), (G.U16, 60000), (G.I16, -3000), (G.U32, 4000000000), (G.I32, -123456),
           (G.F32, 1.5), (G.BOOL, True), (G.U64, 2 ** 63 + 5), (G.I64, -(2 ** 40)), (G.F64, -2.25)]


def rand_bytes(seed, n):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


def tensors_for(seed):
    # (name, type, ne, data): the five matvec types, float types, a 3-D expert stack, a type the matvecs do not
    # take (Q3_K, 11), a 1-D vector
    spec = [("blk.0.ffn_gate.weight", 12, (512, 6)), ("blk.0.ffn_down.weight", 14, (256, 3)),
            ("blk.0.attn_q.weight", 8, (64, 5)), ("blk.0.ffn_up_exps.weight", 100, (64, 3, 4)),
            ("blk.0.ffn_gate_exps.weight", 101, (128, 2, 2)), ("blk.0.attn_norm.weight", 0, (33,)),
            ("token_embd.weight", 1, (16, 7)), ("output.weight", 30, (8, 3)), ("blk.1.q3k.weight", 11, (256, 2))]
    geo = {12: (256, 144), 14: (256, 210), 8: (32, 34), 100: (32, 18), 101: (32, 17), 0: (1, 4), 1: (1, 2),
           30: (1, 2), 11: (256, 110)}
    out = []
    for i, (name, t, ne) in enumerate(spec):
        b, s = geo[t]
        n = int(np.prod(ne))
        out.append((name, t, ne, rand_bytes(seed + i, -(-n // b) * s)))
    return out


def kvs_for():
    kv = [("general.architecture", G.STRING, "qwen3"), ("qwen3.block_count", G.U32, 36),
          ("qwen3.attention.head_count", G.U32, 32), ("qwen3.attention.head_count_kv", G.U16, 8),
          ("qwen3.context_length", G.U64, 40960), ("qwen3.embedding_length", G.I32, 2560),
          ("qwen3.rope.freq_base", G.F32, 1e6), ("qwen3.norm_eps", G.F64, 1e-6),
          ("tokenizer.ggml.model", G.STRING, "gpt2"), ("tokenizer.ggml.pre", G.STRING, "qwen2"),
          ("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, ["a", "bb", "", "é"])),
          ("tokenizer.ggml.token_type", G.ARRAY, (G.I32, [1, 2, 3, -4])),
          ("tokenizer.ggml.scores", G.ARRAY, (G.F32, [0.5, -1.0])), ("empty.array", G.ARRAY, (G.U8, [])),
          ("tokenizer.ggml.vocab_size", G.U32, 151936)]
    kv += [(f"s.{i}", t, v) for i, (t, v) in enumerate(SCALARS)]
    return kv


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("gguf")
    out = {}
    p = d / "m.gguf"
    out["plain"] = (p, G.write(p, kvs_for(), tensors_for(1)), tensors_for(1), 32)
    p = d / "m128.gguf"
    out["align128"] = (p, G.write(p, kvs_for(), tensors_for(2), alignment=128), tensors_for(2), 128)
    return out


def both(ref, path):
    mine = G.Model(path)
    theirs = G.Model(path, ref.ref()) if ref is not None else None
    return mine, theirs


def introspect(m):
    L, h = m.L, m.h
    out = dict(n_t=L.gguf_n_tensors(h), n_kv=L.gguf_n_kv(h), align=L.gguf_alignment(h), off=L.gguf_data_offset(h),
               ver=L.gguf_version(h), arch=L.gguf_arch(h), vocab=L.gguf_vocab_name(h), tok=L.gguf_tokenizer_type(h),
               pre=L.gguf_pre_type(h), vs=L.gguf_vocab_size(h), hc=L.gguf_head_count(h),
               hckv=L.gguf_head_count_kv(h), ctx=L.gguf_context_length(h), emb=L.gguf_embedding_length(h),
               blocks=L.gguf_block_count(h), ai=L.gguf_arch_int(h, b"rope.freq_base", -1),
               af=L.gguf_arch_float(h, b"norm_eps", -1.0), ad=L.gguf_arch_int(h, b"absent", -9),
               nmaps=L.gguf_n_maps(h))
    ts = []
    for i in range(-1, out["n_t"] + 1):
        ne = L.gguf_tensor_ne(h, i)
        n = C.c_size_t()
        name = L.gguf_tensor_name(h, i)
        p = L.gguf_get_tensor_ptr(h, name, C.byref(n)) if 0 <= i < out["n_t"] else None
        base = L.gguf_map_at(h, L.gguf_tensor_split(h, i), None) if 0 <= i < out["n_t"] else None
        ts.append((name, L.gguf_tensor_type(h, i), L.gguf_tensor_dims(h, i), tuple(ne[:4]) if ne else None,
                   L.gguf_tensor_block_size(h, i), L.gguf_tensor_type_size(h, i), L.gguf_tensor_row_size(h, i),
                   L.gguf_tensor_offset(h, i), L.gguf_tensor_nbytes(h, i), L.gguf_tensor_nbytes_pad(h, i),
                   n.value, None if p is None else p - base, L.gguf_tensor_split(h, i)))
    out["tensors"] = ts
    kv = []
    for i in range(-1, out["n_kv"] + 1):
        row = [L.gguf_kv_key(h, i), L.gguf_kv_type(h, i), L.gguf_kv_str_val(h, i)]
        for g in GETTERS:
            row.append(m.get(g, i))
        kv.append(row)
    out["kv"] = kv
    arrays = {}
    for key in (b"tokenizer.ggml.tokens", b"tokenizer.ggml.token_type", b"tokenizer.ggml.scores", b"empty.array",
                b"general.architecture", b"absent"):
        s, n = C.POINTER(C.c_char_p)(), C.c_size_t()
        rc = L.gguf_kv_get_string_array(h, key, C.byref(s), C.byref(n))
        strs = [s[j] for j in range(n.value)] if rc == 0 else None
        t, dp, dn = C.c_int32(), C.c_void_p(), C.c_size_t()
        rc2 = L.gguf_kv_get_array(h, key, C.byref(t), C.byref(dp), C.byref(dn))
        data = C.string_at(dp.value, dn.value * 4) if rc2 == 0 and dn.value and t.value in (4, 5, 6) else None
        arrays[key] = (rc, strs, rc2, t.value if rc2 == 0 else None, dn.value if rc2 == 0 else None, data)
    out["arrays"] = arrays
    return out


@pytest.mark.parametrize("which", ["plain", "align128"])
def test_against_written_values(files, which):
    path, offs, tensors, align = files[which]
    with G.Model(path) as m:
        info = introspect(m)
        L, h = m.L, m.h
        assert info["ver"] == 3 and info["align"] == align and info["off"] % align == 0
        assert info["n_t"] == len(tensors)
        assert info["arch"] == b"qwen3" and info["vocab"] == b"gpt2" and info["pre"] == b"qwen2"
        assert (info["blocks"], info["hc"], info["hckv"], info["ctx"], info["emb"], info["vs"]) == \
            (36, 32, 8, 40960, 2560, 151936)
        assert abs(info["af"] - 1e-6) < 1e-12 and info["ad"] == -9
        base, size = None, C.c_size_t()
        base = L.gguf_map_base(h, C.byref(size))
        assert size.value == os.path.getsize(path)
        for i, (name, t, ne, data) in enumerate(tensors):
            p, n = m.tensor(name)
            assert n == len(data) and C.string_at(p, n) == data
            assert L.gguf_tensor_offset(h, i) == offs[i]
            assert p - base == info["off"] + offs[i]
            assert tuple(L.gguf_tensor_ne(h, i)[:4]) == tuple(ne) + (0,) * (4 - len(ne))
        # string and numeric arrays, in place
        a = info["arrays"]
        assert a[b"tokenizer.ggml.tokens"][1] == [b"a", b"bb", b"", "é".encode()]
        assert np.array_equal(np.frombuffer(a[b"tokenizer.ggml.token_type"][5], np.int32), [1, 2, 3, -4])
        assert a[b"empty.array"][2:5] == (0, 0, 0)
        assert a[b"general.architecture"][0] == -1 and a[b"absent"][0] == -1


def widened(getter, t, v):
    """the value the reference's gguf_kv_get_<getter> gives for a stored (type, value), or None (-1)"""
    bits = {G.U8: 8, G.I8: 8, G.U16: 16, G.I16: 16, G.U32: 32, G.I32: 32, G.U64: 64, G.I64: 64}

    def wrap(x, n, signed):
        x &= (1 << n) - 1
        return x - (1 << n) if signed and x >> (n - 1) else x
    ints = {G.U8, G.I8, G.U16, G.I16, G.U32, G.I32}
    if getter == "f32":
        return float(np.float32(v)) if t == G.F32 else None
    if getter == "f64":
        return float(np.float32(v)) if t == G.F32 else (v if t == G.F64 else None)
    accept = {"u8": {G.U8, G.I8, G.BOOL}, "i8": {G.U8, G.I8}, "u16": {G.U8, G.I8, G.U16, G.I16},
              "i16": {G.U8, G.I8, G.U16, G.I16}, "u32": ints, "i32": ints, "u64": ints | {G.U64},
              "i64": ints | {G.U64, G.I64}}[getter]
    if t not in accept:
        return None
    if t == G.BOOL:
        return 1 if v else 0
    n, signed = int(getter[1:]), getter[0] == "i"
    if getter == "u64" and t == G.I8:
        return v & 0xff  # (the reference zero-extends an int8 into u64)
    return wrap(v, n, signed)


def test_getter_widening_rules(files):
    path = files["plain"][0]
    with G.Model(path) as m:
        for i, (t, v) in enumerate(SCALARS):
            idx = m.kv_index(f"s.{i}")
            assert m.L.gguf_kv_type(m.h, idx) == t
            for g in GETTERS:
                rc, got = m.get(g, idx)
                want = widened(g, t, v)
                assert (rc == 0) == (want is not None), (g, t)
                if want is not None:
                    assert got == want, (g, t, got, want)
        # strings and arrays take no scalar getter; kv_type of an array is its element type
        for key, et in (("tokenizer.ggml.tokens", G.STRING), ("tokenizer.ggml.token_type", G.I32)):
            idx = m.kv_index(key)
            assert m.L.gguf_kv_type(m.h, idx) == et
            assert all(m.get(g, idx)[0] == -1 for g in GETTERS)


@pytest.mark.parametrize("which", ["plain", "align128"])
def test_same_answers_as_the_reference_reader(ref, files, which):
    path = files[which][0]
    mine, theirs = both(ref, path)
    try:
        a, b = introspect(mine), introspect(theirs)
        for k in a:
            assert a[k] == b[k], k
    finally:
        mine.close()
        theirs.close()


def write_split(d, n_parts, seed):
    tensors = tensors_for(seed)
    per = -(-len(tensors) // n_parts)
    paths = []
    for i in range(n_parts):
        p = d / f"sm-{i + 1:05d}-of-{n_parts:05d}.gguf"
        kv = ([("general.architecture", G.STRING, "llama"), ("llama.block_count", G.U32, 2)] if i == 0 else [])
        kv += [("split.no", G.U16, i), ("split.count", G.U16, n_parts)]
        G.write(p, kv, tensors[i * per:(i + 1) * per], alignment=64 if i % 2 else None)
        paths.append(p)
    return paths, tensors, per


@pytest.mark.parametrize("n_parts", [2, 3])
def test_split_model(ref, tmp_path, n_parts):
    paths, tensors, per = write_split(tmp_path, n_parts, 40 + n_parts)
    mine, theirs = both(ref, paths[0])
    try:
        L, h = mine.L, mine.h
        assert L.gguf_n_maps(h) == n_parts and L.gguf_n_tensors(h) == len(tensors)
        assert L.gguf_block_count(h) == 2
        for i, (name, t, ne, data) in enumerate(tensors):
            p, n = mine.tensor(name)
            assert C.string_at(p, n) == data
            assert L.gguf_tensor_split(h, i) == i // per
            assert L.gguf_file_path(h, i // per).decode() == str(paths[i // per])
        ida, idb = (C.c_uint64 * 4)(), (C.c_uint64 * 4)()
        for i in range(n_parts):
            assert L.gguf_file_identity(h, i, ida) == 0 == theirs.L.gguf_file_identity(theirs.h, i, idb)
            assert list(ida) == list(idb) and ida[2] == os.path.getsize(paths[i])
        a, b = introspect(mine), introspect(theirs)
        for k in a:
            assert a[k] == b[k], k
    finally:
        mine.close()
        theirs.close()
    # opened by another part than the first, or with a part missing: refused
    assert not G.lib().gguf_mmap_open(str(paths[1]).encode())
    os.rename(paths[-1], str(paths[-1]) + ".x")
    assert not G.lib().gguf_mmap_open(str(paths[0]).encode())


def test_long_names_truncate_as_the_reference(ref, tmp_path):
    long = "blk.0." + "x" * 80 + ".weight"
    p = tmp_path / "long.gguf"
    G.write(p, [], [(long, 0, (4,), b"\1" * 16)])
    mine, theirs = both(ref, p)
    try:
        assert mine.names() == theirs.names() == [long[:63]]
        assert mine.tensor(long[:63])[1] == 16 and mine.tensor(long)[0] is None
    finally:
        mine.close()
        theirs.close()


def test_malformed_files_are_refused(files, tmp_path):
    data = open(files["plain"][0], "rb").read()
    L = G.lib()

    def opens(blob, name):
        p = tmp_path / name
        p.write_bytes(blob)
        h = L.gguf_mmap_open(str(p).encode())
        if h:
            L.gguf_mmap_close(h)
        return bool(h)
    assert opens(data, "ok.gguf")
    # every cut through the header, the key/values or the tensor table, and cuts into the data
    hdr_end = G.Model(files["plain"][0]).L.gguf_data_offset(G.Model(files["plain"][0]).h)
    cuts = sorted(set(list(range(0, 64)) + list(range(64, hdr_end, 7)) + [hdr_end, len(data) - 1]))
    for n in cuts:
        assert not opens(data[:n], f"cut{n}.gguf"), n
    assert not opens(b"GGUX" + data[4:], "magic.gguf")
    assert not opens(data[:4] + struct.pack("<I", 2) + data[8:], "v2.gguf")
    # n_dims 0 and 5, a nested array, a non-power-of-two alignment, an unknown key type
    assert not opens(bytes(_table_with_dims(0)), "d0.gguf") and not opens(bytes(_table_with_dims(5)), "d5.gguf")
    nested = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + G._s(b"k") + struct.pack("<IIQ", G.ARRAY, G.ARRAY, 0)
    assert not opens(nested, "nested.gguf")
    p = tmp_path / "a48.gguf"
    G.write(p, [], [("t", 0, (4,), b"\0" * 16)], alignment=48)
    assert not L.gguf_mmap_open(str(p).encode())
    bad = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + G._s(b"k") + struct.pack("<I", 13) + b"\0" * 16
    assert not opens(bad, "ktype.gguf")


def _table_with_dims(nd):
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, 1, 0))
    out += G._s(b"t") + struct.pack("<I", nd) + struct.pack(f"<{nd}Q", *([4] * nd)) + struct.pack("<IQ", 0, 0)
    out += b"\0" * ((-len(out)) % 32) + b"\0" * 4096
    return out


def test_bind_weight_and_hbm_bytes(files):
    path, offs, tensors, align = files["plain"]
    with G.Model(path) as m:
        rc, w = m.bind_weight("blk.0.ffn_gate.weight")
        assert rc == 0 and (w.type, w.N, w.K, w.row_bytes) == (12, 6, 512, 288)
        rc, w = m.bind_weight("blk.0.ffn_up_exps.weight")  # 3-D: experts stacked as rows
        assert rc == 0 and (w.type, w.N, w.K, w.row_bytes) == (100, 12, 64, 36)
        assert m.bind_weight("blk.0.attn_norm.weight")[0] == 0  # F32 vector: one row
        assert m.bind_weight("blk.1.q3k.weight")[0] == -1       # a type the matvecs do not take
        assert m.bind_weight("absent.weight")[0] == 1
        sizes = [len(d) for _, _, _, d in tensors]
        want = 0
        for s in sizes:
            want = -(-want // 256) * 256 + s
        assert m.hbm_bytes() == want
        keep = np.zeros(len(tensors), np.uint8)
        keep[[0, 3]] = 1
        assert m.hbm_bytes(keep) == -(-sizes[0] // 256) * 256 + sizes[3]


def test_remap_and_staging_hooks(files):
    path = files["plain"][0]
    with G.Model(path) as m:
        L, h = m.L, m.h
        size = C.c_size_t()
        base = L.gguf_map_base(h, C.byref(size))
        page = os.sysconf("SC_PAGE_SIZE")
        before = C.string_at(base, page)
        assert L.gguf_remap(h, base, page) == 0 and C.string_at(base, page) == before
        assert L.gguf_remap(h, base + 1, page) == -1 and L.gguf_remap(h, base, 3) == -1
        src = L.gguf_tensor_source(h, 2)
        buf = C.create_string_buffer(b"\7" * 64)
        L.gguf_set_tensor_staged(h, 2, C.cast(buf, C.c_void_p))
        name = L.gguf_tensor_name(h, 2).decode()
        assert m.tensor(name)[0] == C.addressof(buf) and L.gguf_tensor_source(h, 2) == src
        L.gguf_set_tensor_staged(h, 2, None)
        assert m.tensor(name)[0] == src
        assert L.gguf_type_is_self_contained(12) == 1
