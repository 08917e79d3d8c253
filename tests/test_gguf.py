"""GGUF catalog and layer-pack loader (host side; no GPU).

The reference's own GGUF tests (crates/hayai-model/src/gguf.rs:813-886) restated against
the C-ABI catalog, the parse rules of parse_header_bytes (gguf.rs:25-127) and read_value
(:633-676) on malformed files, tensor_nbytes (:240-284), and the layout and bytes of
load_layer_pack_into (gguf_stream.rs:451-638) on files written by hayai_amd.gguf.write_gguf,
through io_uring and through positioned reads.
"""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

import hayai_amd
from hayai_amd import gguf
from hayai_amd.gguf import GgufCatalog, write_gguf

HERE = os.path.dirname(os.path.abspath(__file__))


def _err(fn, *a):
    with pytest.raises(hayai_amd.HipError) as e:
        fn(*a)
    return e.value


def test_roundtrip_minimal_gguf(tmp_path):
    # gguf.rs:813-833
    p = str(tmp_path / "minimal.gguf")
    data = np.ones(32, np.float32)
    write_gguf(p, [("general.architecture", "llama"), ("llama.embedding_length", (gguf.U32, 8))],
               [("token_embd.weight", (8, 4), 0, data)])
    with GgufCatalog(p) as g:
        assert g.meta_str("general.architecture") == "llama"
        assert g.meta_u32("llama.embedding_length") == 8
        t = g.tensor("token_embd.weight")
        assert (t.dims, t.type, t.nbytes, t.ncols, t.nrows) == ((8, 4), 0, 128, 8, 4)
        np.testing.assert_array_equal(g.read_tensor("token_embd.weight").view(np.float32), data)
        assert g.version == 3 and g.alignment == 32 and g.data_offset % 32 == 0


def test_zero_alignment_is_rejected(tmp_path):
    # gguf.rs:840-853
    p = str(tmp_path / "zero_align.gguf")
    write_gguf(p, [("general.alignment", (gguf.U32, 0))], [("t.weight", (4,), 0, np.zeros(4, np.float32))])
    e = _err(GgufCatalog, p)
    assert "alignment" in str(e)


def test_duplicate_tensor_names_are_rejected(tmp_path):
    # gguf.rs:855-872
    p = str(tmp_path / "dup.gguf")
    z = np.zeros(4, np.float32)
    write_gguf(p, [], [("t.weight", (4,), 0, z), ("t.weight", (4,), 0, z)])
    assert "duplicate" in str(_err(GgufCatalog, p))


def test_tensor_nbytes_overflow_is_rejected():
    # gguf.rs:874-885
    _err(gguf.tensor_nbytes, 0, (2**64 - 1, 2))


@pytest.mark.parametrize("t,block,bb", [
    (0, 1, 4), (1, 1, 2), (30, 1, 2), (28, 1, 8), (27, 1, 8), (24, 1, 1), (25, 1, 2), (26, 1, 4),
    (2, 32, 18), (3, 32, 20), (6, 32, 22), (7, 32, 24), (8, 32, 34), (9, 32, 36), (20, 32, 18),
    (10, 256, 84), (11, 256, 110), (12, 256, 144), (13, 256, 176), (14, 256, 210), (15, 256, 292),
    (16, 256, 66), (17, 256, 74), (22, 256, 82), (18, 256, 98), (21, 256, 110), (19, 256, 50),
    (29, 256, 56), (23, 256, 136), (34, 256, 54), (35, 256, 66)])
def test_tensor_nbytes_table(t, block, bb):
    # ceil(elements / block) * block bytes, elements the product of the dims
    for dims in ((4096, 14336), (576,), (7, 3, 2), (block * 3 + 1,)):
        n = int(np.prod(dims))
        assert gguf.tensor_nbytes(t, dims) == -(-n // block) * bb
    _err(gguf.tensor_nbytes, 99, (256,))  # unknown type id


def _header(version=3, n_tensors=0, n_kv=0):
    return struct.pack("<IIQQ", gguf.GGUF_MAGIC, version, n_tensors, n_kv)


def _kv(key, ty, payload):
    return struct.pack("<Q", len(key)) + key.encode() + struct.pack("<I", ty) + payload


def _write(tmp_path, name, blob):
    p = str(tmp_path / name)
    with open(p, "wb") as f:
        f.write(blob)
    return p


def test_malformed_headers_are_rejected(tmp_path):
    cases = {
        "bad_magic": (struct.pack("<IIQQ", 0x46554748, 3, 0, 0), "magic"),
        "version0": (_header(version=0), "version"),
        "version5": (_header(version=5), "version"),
        "unknown_meta_type": (_header(n_kv=1) + _kv("k", 13, b"\0" * 8), "unknown metadata type"),
        "huge_kv_count": (struct.pack("<IIQQ", gguf.GGUF_MAGIC, 3, 0, 2**40), "truncated"),
        "huge_tensor_count": (struct.pack("<IIQQ", gguf.GGUF_MAGIC, 3, 2**40, 0), "truncated"),
        "five_dims": (_header(n_tensors=1) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 5) +
                      struct.pack("<5Q", 1, 1, 1, 1, 1) + struct.pack("<IQ", 0, 0), "5 dims"),
        "zero_dim": (_header(n_tensors=1) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 2) +
                     struct.pack("<2Q", 4, 0) + struct.pack("<IQ", 0, 0), "zero dimension"),
        "unsupported_type": (_header(n_tensors=1) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 1) +
                             struct.pack("<Q", 256) + struct.pack("<IQ", 99, 0), "type"),
        "align48": (_header(n_kv=1) + _kv("general.alignment", gguf.U32, struct.pack("<I", 48)), "alignment"),
        "offset_overflow": (_header(n_tensors=1) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 1) +
                            struct.pack("<Q", 4) + struct.pack("<IQ", 0, 2**64 - 8), "overflow"),
    }
    for name, (blob, what) in cases.items():
        e = _err(GgufCatalog, _write(tmp_path, name + ".gguf", blob))
        assert what in str(e), (name, str(e))


def test_nested_arrays_beyond_depth_32_are_rejected(tmp_path):
    def nested(depth):
        v = struct.pack("<IQ", gguf.U8, 0)  # innermost: empty u8 array
        for _ in range(depth):
            v = struct.pack("<IQ", gguf.ARRAY, 1) + v
        return v
    ok = _write(tmp_path, "d32.gguf", _header(n_kv=1) + _kv("a", gguf.ARRAY, nested(31)))
    GgufCatalog(ok).close()
    e = _err(GgufCatalog, _write(tmp_path, "d34.gguf", _header(n_kv=1) + _kv("a", gguf.ARRAY, nested(33))))
    assert "nesting" in str(e)


def test_truncated_files_fail_cleanly(tmp_path):
    p = str(tmp_path / "full.gguf")
    write_gguf(p, [("general.architecture", "llama"), ("arr", (gguf.ARRAY, (gguf.STRING, ["a", "bb", "ccc"])))],
               [("a.weight", (256, 2), 12, np.arange(288, dtype=np.uint8)),
                ("b.weight", (32,), 8, np.arange(34, dtype=np.uint8))])
    blob = open(p, "rb").read()
    with GgufCatalog(p) as g:
        end = g.header_bytes
    # any cut inside the header and directory fails to open (the parse needs every byte)
    for cut in sorted({0, 3, 8, 20, 24, 40, end // 2, end - 1}):
        q = _write(tmp_path, f"cut{cut}.gguf", blob[:cut])
        _err(GgufCatalog, q)
    # a directory that points past the end of the file opens, but reading the tensor fails
    q = _write(tmp_path, "short_data.gguf", blob[:-10])
    with GgufCatalog(q) as g:
        e = _err(g.read_tensor, "b.weight")
        assert e.status == 7  # HH_ERR_IO


def test_metadata_accessors_follow_as_u64_as_u32(tmp_path):
    p = str(tmp_path / "meta.gguf")
    write_gguf(p, [("u8", (gguf.U8, 7)), ("u16", (gguf.U16, 300)), ("u32", (gguf.U32, 70000)),
                   ("u64", (gguf.U64, 2**40)), ("i32n", (gguf.I32, -5)), ("i32", (gguf.I32, 12)),
                   ("i64", (gguf.I64, 2**35)), ("f32", (gguf.F32, 0.5)), ("f64", (gguf.F64, 0.25)),
                   ("s", "hi"), ("b", True), ("arr", (gguf.ARRAY, (gguf.U32, [1, 2, 3])))], [])
    with GgufCatalog(p) as g:
        assert g.n_metadata == 12
        # as_u32: U8/U16/U32 always, U64/I32/I64 when they fit
        assert [g.meta_u32(k) for k in ("u8", "u16", "u32", "u64", "i32n", "i32", "i64")] == \
            [7, 300, 70000, None, None, 12, None]
        # as_u64: U64, U32, non-negative I32/I64 only (not U8/U16)
        assert [g.meta_u64(k) for k in ("u8", "u16", "u32", "u64", "i32n", "i32", "i64")] == \
            [None, None, 70000, 2**40, None, 12, 2**35]
        assert (g.meta_f32("f32"), g.meta_f32("f64"), g.meta_f32("u32")) == (0.5, 0.25, None)
        assert (g.meta_str("s"), g.meta_str("u8"), g.meta_str("missing")) == ("hi", None, None)
        assert g.meta_u32("arr") is None


def test_custom_alignment_places_the_data_section(tmp_path):
    p = str(tmp_path / "a64.gguf")
    offs = write_gguf(p, [], [("x.weight", (32,), 2, np.arange(18, dtype=np.uint8)),
                              ("y.weight", (32,), 2, np.arange(18, 36, dtype=np.uint8))], alignment=64)
    assert offs == [0, 64]
    with GgufCatalog(p) as g:
        assert g.alignment == 64 and g.data_offset % 64 == 0
        assert [t.offset for t in g.tensors()] == [0, 64]
        np.testing.assert_array_equal(g.read_tensor("y.weight"), np.arange(18, 36, dtype=np.uint8))


def _rand(rng, nbytes):
    return rng.integers(0, 256, nbytes, dtype=np.uint8)


def _model(tmp_path, rng, layers=2, fused=None, no_v=False, attn_gate_layer=None, drop=None):
    """A Llama-like file: per layer attn q/k/v/o (F16, Q8_0), ffn gate/up Q4_K, down Q6_K."""
    dm, dff, kv = 512, 1024, 128
    tensors, want = [], {}
    for l in range(layers):
        spec = [("attn_q", (dm, dm), 1), ("attn_k", (dm, kv), 8), ("attn_v", (dm, kv), 8),
                ("attn_output", (dm, dm), 12)]
        if fused == "gate_up":
            spec += [("ffn_gate_up", (dm, 2 * dff), 12)]
        elif fused == "phi3":
            spec += [("ffn_up", (dm, 2 * dff), 12)]
        else:
            spec += [("ffn_gate", (dm, dff), 12), ("ffn_up", (dm, dff), 12)]
        spec += [("ffn_down", (dff, dm), 14)]
        if attn_gate_layer == l:
            spec += [("attn_gate", (dm, dm), 2)]
        for name, dims, ty in spec:
            if (no_v and name == "attn_v") or (drop and name == drop):
                continue
            full = f"blk.{l}.{name}.weight"
            b = _rand(rng, gguf.tensor_nbytes(ty, dims))
            tensors.append((full, dims, ty, b))
            want[full] = (dims, ty, b)
    tensors.append(("output_norm.weight", (dm,), 0, np.ones(dm, np.float32)))
    p = str(tmp_path / "model.gguf")
    write_gguf(p, [("general.architecture", "llama")], tensors)
    return p, want


@pytest.mark.parametrize("force_file", [False, True])
def test_layer_pack_layout_and_bytes(tmp_path, force_file, monkeypatch):
    if force_file:
        monkeypatch.setenv("HAYAI_FORCE_FILE_IO", "1")
    rng = np.random.default_rng(0)
    p, want = _model(tmp_path, rng, layers=3, attn_gate_layer=1)
    with GgufCatalog(p) as g:
        if force_file:
            assert not g.io_uring
        for l in range(3):
            lp = g.layer_pack(l)
            names = [f"blk.{l}.{s}.weight" for s in gguf.SLOTS]
            off = 0
            for i, n in enumerate(names):
                if n not in want:
                    assert lp.len[i] == 0
                    continue
                dims, ty, b = want[n]
                assert (lp.off[i], lp.len[i], lp.type[i], lp.cols[i], lp.rows[i]) == (off, b.size, ty, dims[0], dims[1])
                off += b.size
            assert lp.total == off and not lp.fused_gate_up
            dst = np.full(lp.total + 100, 0xAB, np.uint8)
            lp2 = g.load_layer_pack(l, dst)
            assert lp2 == lp
            for i, n in enumerate(names):
                if n in want:
                    np.testing.assert_array_equal(dst[lp.off[i]:lp.off[i] + lp.len[i]], want[n][2])
            assert (dst[lp.total:] == 0xAB).all()  # nothing written past the pack
            e = _err(g.load_layer_pack, l, np.zeros(lp.total - 1, np.uint8))
            assert "exceeds" in str(e)


@pytest.mark.parametrize("fused", ["gate_up", "phi3"])
def test_layer_pack_fused_gate_up_splits_rows(tmp_path, fused):
    rng = np.random.default_rng(1)
    p, want = _model(tmp_path, rng, layers=1, fused=fused)
    with GgufCatalog(p) as g:
        lp = g.layer_pack(0)
        assert lp.fused_gate_up
        src = want["blk.0.ffn_gate_up.weight" if fused == "gate_up" else "blk.0.ffn_up.weight"][2]
        half = src.size // 2
        assert lp.len[4] == lp.len[5] == half and lp.off[5] == lp.off[4] + half
        assert lp.rows[4] == lp.rows[5] == 1024 and lp.cols[4] == lp.cols[5] == 512
        dst = np.zeros(lp.total, np.uint8)
        g.load_layer_pack(0, dst)
        np.testing.assert_array_equal(dst[lp.off[4]:lp.off[4] + half], src[:half])
        np.testing.assert_array_equal(dst[lp.off[5]:lp.off[5] + half], src[half:])


def test_layer_pack_optional_and_missing_tensors(tmp_path):
    rng = np.random.default_rng(2)
    p, _ = _model(tmp_path, rng, layers=1, no_v=True)
    with GgufCatalog(p) as g:
        lp = g.layer_pack(0)
        assert lp.len[2] == 0 and lp.off[2] == lp.off[3]  # V = K layer
        e = _err(g.layer_pack, 1)  # no such layer
        assert e.status == 8
    p, _ = _model(tmp_path, rng, layers=1, drop="ffn_down")
    with GgufCatalog(p) as g:
        e = _err(g.layer_pack, 0)
        assert e.status == 8 and "ffn_down" in str(e)
    p, _ = _model(tmp_path, rng, layers=1, drop="ffn_gate")
    with GgufCatalog(p) as g:  # ungated FFN: an empty gate region
        lp = g.layer_pack(0)
        assert lp.len[4] == 0 and not lp.fused_gate_up


def test_catalog_reads_are_identical_through_io_uring_and_pread(tmp_path):
    rng = np.random.default_rng(3)
    p, _ = _model(tmp_path, rng, layers=2)
    out = []
    for force in ("0", "1"):
        code = ("import numpy as np, sys; from hayai_amd.gguf import GgufCatalog; g = GgufCatalog(sys.argv[1]); "
                "lp = g.layer_pack(1); d = np.zeros(lp.total, np.uint8); g.load_layer_pack(1, d); "
                "print(int(g.io_uring), d.sum(dtype=np.uint64), d[::997].tobytes().hex())")
        env = dict(os.environ, HAYAI_FORCE_FILE_IO=force)
        r = subprocess.run([sys.executable, "-c", code, p], env=env, capture_output=True, text=True,
                           cwd=os.path.dirname(HERE), timeout=120)
        assert r.returncode == 0, r.stderr
        out.append(r.stdout.split())
    assert out[1][0] == "0"
    assert out[0][1:] == out[1][1:]


@pytest.mark.parametrize("tail", [0, 123])
def test_o_direct_reads_are_identical(tmp_path, tail):
    # HAYAI_O_DIRECT (weight_io.rs:243-263,329-405): runs read as their 4096-aligned cover
    # through O_DIRECT and copied out; identical bytes to page-cache reads.  A file whose
    # size is not a multiple of 4096 (tail > 0) sends the run that reaches its end back to
    # page-cache reads, for good; a filesystem that refuses O_DIRECT (tmpfs) does the same
    # from the start.
    rng = np.random.default_rng(4)
    p, _ = _model(tmp_path, rng, layers=2)
    with open(p, "ab") as f:  # pad to a 4096 multiple, then `tail` more bytes
        f.write(b"\0" * ((-os.path.getsize(p)) % 4096 + tail))
    out = []
    for env_extra in ({}, {"HAYAI_O_DIRECT": "1"}, {"HAYAI_O_DIRECT": "1", "HAYAI_FORCE_FILE_IO": "1"}):
        code = ("import numpy as np, sys; from hayai_amd.gguf import GgufCatalog; g = GgufCatalog(sys.argv[1]); "
                "d0 = int(g.o_direct); r = []\n"
                "for l in (1, 0, 1):\n"
                "    lp = g.layer_pack(l); d = np.zeros(lp.total, np.uint8); g.load_layer_pack(l, d)\n"
                "    r.append(d.sum(dtype=np.uint64)); r.append(d[::991].tobytes().hex())\n"
                "print(d0, *r)")
        env = dict(os.environ, **env_extra)
        env.pop("HAYAI_O_DIRECT", None) if not env_extra else None
        r = subprocess.run([sys.executable, "-c", code, p], env=env, capture_output=True, text=True,
                           cwd=os.path.dirname(HERE), timeout=120)
        assert r.returncode == 0, r.stderr
        out.append(r.stdout.split())
    assert out[0][0] == "0"
    assert out[0][1:] == out[1][1:] == out[2][1:]


def test_mutated_headers_never_crash(tmp_path):
    # 300 files, each a valid header with a few random bytes changed (or cut short): opening
    # either succeeds with a self-consistent directory or fails with a status; a successful
    # open's tensors all lie inside 64-bit ranges and reading them either works or reports
    # HH_ERR_IO / HH_ERR_INVALID.
    rng = np.random.default_rng(123)
    p = str(tmp_path / "base.gguf")
    write_gguf(p, [("general.architecture", "llama"), ("n", (gguf.U32, 7)),
                   ("arr", (gguf.ARRAY, (gguf.I32, [1, -2, 3]))), ("s", "abc")],
               [("a.weight", (256, 2), 12, np.arange(288, dtype=np.uint8)),
                ("b.weight", (32, 3), 8, np.arange(102, dtype=np.uint8))])
    blob = bytearray(open(p, "rb").read())
    with GgufCatalog(p) as g:
        hdr = g.header_bytes
    opened = 0
    for i in range(300):
        b = bytearray(blob)
        for _ in range(int(rng.integers(1, 4))):
            pos = int(rng.integers(0, hdr))
            b[pos] = int(rng.integers(0, 256))
        if i % 10 == 0:
            b = b[: int(rng.integers(0, len(b)))]
        q = str(tmp_path / f"m{i}.gguf")
        with open(q, "wb") as f:
            f.write(b)
        try:
            g = GgufCatalog(q)
        except hayai_amd.HipError as e:
            assert e.status in (2, 3, 7), e  # invalid / unknown type / io
            continue
        opened += 1
        with g:
            for t in g.tensors():
                assert t.abs_offset == g.data_offset + t.offset
                if t.nbytes <= 1 << 20:
                    try:
                        g.read_tensor(t.name)
                    except hayai_amd.HipError as e:
                        assert e.status in (2, 7), e
    assert opened > 0


def test_names_are_decoded_like_from_utf8_lossy(tmp_path):
    # String::from_utf8_lossy (gguf.rs:620-626): each maximal prefix of an invalid sequence ->
    # one U+FFFD; Python's "replace" handler follows the same rule, so it is the reference here.
    raws = [b"ok.weight", b"t\xff.weight", b"e\xe2\x82A", b"s\xed\xa0\x80x", b"f\xf0\x9f\x98\x80y", b"c\xc0\xafz",
            b"tail\xe2\x82"]
    p = str(tmp_path / "names.gguf")
    write_gguf(p, [], [(r, (32,), 8, np.zeros(34, np.uint8)) for r in raws])
    with GgufCatalog(p) as g:
        names = [t.name for t in g.tensors()]
        assert names == [r.decode("utf-8", "replace") for r in raws]
        for n in names:
            assert g.tensor(n).nbytes == 34
