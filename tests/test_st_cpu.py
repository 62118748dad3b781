"""Checkpoint index (dsv4g_st_*) on the CPU: no GPU call is made.

The index is checked three ways: against the reference reader k3_st
(src/io/k3_st.c, compiled in oracle/_ref) on the same directories, against an
independent parse with Python's json module, and against the reference's own
fixtures (tests/fixtures/st, tests/fixtures/tiny_dsv4, copied as data into
tests/golden/) with the known answers of tests/unit/test_dsv4_st.c:20-45.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np
import pytest

from common import ROOT, write_safetensors, write_checkpoint
import pyoracle

from dsv4_gpu import Checkpoint, DTYPE_CODES, GpuLib, LIB_PATH

GOLD = os.path.join(ROOT, "tests", "golden")
ST_DIR = os.path.join(GOLD, "st")
TINY_DIR = os.path.join(GOLD, "tiny_dsv4")

pytestmark = pytest.mark.skipif(not os.path.exists(LIB_PATH), reason="library not built")


@pytest.fixture(scope="module")
def gl():
    return GpuLib()


def ref_st(directory):
    if not pyoracle.ref_available():
        return None
    return pyoracle.RefSt(pyoracle.RefLib(), directory)


def py_index(directory):
    """Independent index: json.loads of each sorted *.safetensors header."""
    files = sorted(f for f in os.listdir(directory) if f.endswith(".safetensors"))
    out = []
    for k, f in enumerate(files):
        with open(os.path.join(directory, f), "rb") as fh:
            n = struct.unpack("<Q", fh.read(8))[0]
            hdr = json.loads(fh.read(n).decode("utf-8"))
        for name, v in hdr.items():
            if name == "__metadata__":
                continue
            o0, o1 = v["data_offsets"]
            out.append(dict(name=name, shard=k, dtype=DTYPE_CODES[v["dtype"]],
                            shape=tuple(v["shape"]), off=8 + n + o0, nbytes=o1 - o0))
    return out


def ascii_names(idx):
    """The reference keeps ASCII from \\u escapes and turns the rest into '?'."""
    return [dict(t, name="".join(c if ord(c) < 128 else "?" for c in t["name"])) for t in idx]


def file_bytes(directory, shard_path, t):
    with open(shard_path, "rb") as f:
        f.seek(t["off"])
        return f.read(t["nbytes"])


def widen(raw, dtype):
    """Host widening rule of k3_st_read_f32 (src/io/k3_st.c:566-597) from
    numpy's own conversions: byte dtypes give their raw code as a number."""
    if dtype == DTYPE_CODES["F32"]:
        return np.frombuffer(raw, np.float32)
    if dtype == DTYPE_CODES["BF16"]:
        return (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32)
    if dtype == DTYPE_CODES["F16"]:
        return np.frombuffer(raw, np.float16).astype(np.float32)
    if dtype == DTYPE_CODES["I64"]:
        return np.frombuffer(raw, np.int64).astype(np.float32)
    return np.frombuffer(raw, np.uint8).astype(np.float32)


def check_directory(gl, directory):
    ck = Checkpoint(directory, gl)
    ours = ck.tensors()
    assert ours == ascii_names(py_index(directory))
    ref = ref_st(directory)
    if ref is not None:
        assert ref.ok
        assert ref.nshard() == ck.nshard()
        assert ref.tensors() == ours
    for t in ours:
        assert ck.find(t["name"]) == t
        raw = ck.read(t["name"])
        assert raw == file_bytes(directory, ck.shard_path(t["shard"]), t)
        wide = ck.read_f32(t["name"])
        want = widen(raw, t["dtype"])
        assert wide.view(np.uint32).tolist() == want.view(np.uint32).tolist(), t["name"]
        if ref is not None:
            assert ref.read(t["name"]) == raw
            assert ref.read_f32(t["name"]).view(np.uint32).tolist() == \
                wide.view(np.uint32).tolist()
    return ck, ours


def test_reference_fixture_known_answers(gl):
    """tests/unit/test_dsv4_st.c:20-45 on the fixture shards, plus the
    fixture's edge cases: metadata skipped, scalar, empty, rank 3/4, escaped
    name on the second shard."""
    ck, ours = check_directory(gl, ST_DIR)
    assert ck.nshard() == 2
    names = [t["name"] for t in ours]
    assert "__metadata__" not in names
    assert len(names) == 13
    t = ck.find("plain.f32.2d")
    assert t["dtype"] == DTYPE_CODES["F32"] and t["shape"] == (16, 16)
    v = ck.read_f32("plain.f32.2d")
    assert v.size == 256 and v[0] != 0 and v[255] != 0
    b = ck.find("plain.bf16.1d")
    assert b["dtype"] == DTYPE_CODES["BF16"]
    v = ck.read_f32("plain.bf16.1d")
    assert v.size == 128 and v[0] != 0 and v[127] != 0
    assert ck.find("tricky.f16.1d")["dtype"] == DTYPE_CODES["F16"]
    assert ck.find("scalar.f32")["shape"] == () and ck.find("scalar.f32")["nbytes"] == 4
    assert ck.find("empty.f32")["nbytes"] == 0 and ck.read("empty.f32") == b""
    assert ck.find("rank4.u8")["shape"] == (2, 2, 2, 2)
    w = ck.find('weird\\name."with"quotes')
    assert w is not None and w["shard"] == 1 and w["shape"] == (3,)
    assert ck.find("plain.f32") is None and ck.find("") is None


def test_reference_tiny_checkpoint(gl):
    """The reference's tiny DeepSeek-V4 checkpoint (all eight dtypes the
    engine binds, 233 tensors): index, bytes and widening agree."""
    ck, ours = check_directory(gl, TINY_DIR)
    assert len(ours) == 233
    dts = {t["dtype"] for t in ours}
    for d in ("BF16", "F32", "F8_E4M3", "F8_E8M0", "I8"):
        assert DTYPE_CODES[d] in dts
    t = ck.find("layers.0.ffn.experts.3.w2.weight")
    assert t["shape"] == (8, 2) and t["dtype"] == DTYPE_CODES["I8"]


def test_json_forms_and_escapes(gl, tmp_path):
    """Escapes (\\uXXXX ASCII kept, others '?'; \\n \\/ \\"), whitespace,
    unknown keys with nested values, metadata holding brackets in strings,
    entries out of offset order, a trailing comma."""
    d = tmp_path / "esc"
    d.mkdir()
    f32 = np.arange(6, dtype=np.float32)
    body = f32.tobytes() + bytes(range(10))
    hdr = ('{ "__metadata__" : {"a": "}{][\\"", "b": [1, {"c": [2]}]},\n'
           '  "u8.\\u0041\\u00e9\\n\\/x" : {"data_offsets":[24,34], "extra": {"k": [1, [2]]},'
           ' "dtype":"U8", "shape":[10]},\t'
           '"f" : {"shape": [2,3], "dtype": "F32", "data_offsets": [0, 24]},\r\n}')
    h = hdr.encode()
    with open(d / "a.safetensors", "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + body)
    ck = Checkpoint(str(d), gl)
    names = [t["name"] for t in ck.tensors()]
    assert names == ["u8.A?\n/x", "f"]
    assert ck.read("f") == f32.tobytes()
    assert ck.read("u8.A?\n/x") == bytes(range(10))
    ref = ref_st(str(d))
    if ref is not None:
        assert ref.ok and ref.tensors() == ck.tensors()


def test_many_tensors_hash_index(gl, tmp_path):
    """6000 tensors with the checkpoint's long shared prefixes over three
    shards: every name found, absent names not, same index as k3_st."""
    d = str(tmp_path / "many")
    ents = []
    for e in range(1000):
        for m in ("w1", "w2", "w3"):
            for kind, dt in (("scale", "F8_E8M0"), ("weight", "I8")):
                ents.append((f"layers.7.ffn.experts.{e}.{m}.{kind}", dt, (2,), bytes([e % 251, 7])))
    write_checkpoint(d, ents, n_shards=3)
    ck = Checkpoint(d, gl)
    assert len(ck) == 6000 and ck.nshard() == 3
    for name, _, _, raw in ents[::37]:
        assert ck.read(name) == raw
    assert ck.find("layers.7.ffn.experts.1000.w1.scale") is None
    assert ck.find("layers.7.ffn.experts.10.w4.scale") is None
    ref = ref_st(d)
    if ref is not None:
        assert ref.tensors() == ck.tensors()


def test_shards_sorted_and_filtered(gl, tmp_path):
    """Shard numbers follow the sorted file names; other files are ignored."""
    d = tmp_path / "order"
    d.mkdir()
    for nm in ("c", "a", "b"):
        write_safetensors(str(d / f"{nm}.safetensors"), [(f"t.{nm}", "U8", (1,), nm.encode())])
    (d / "config.json").write_text("{}")
    (d / "x.safetensors.tmp").write_bytes(b"junk")
    ck = Checkpoint(str(d), gl)
    assert [t["name"] for t in ck.tensors()] == ["t.a", "t.b", "t.c"]
    assert [ck.find(f"t.{n}")["shard"] for n in "abc"] == [0, 1, 2]
    assert ck.read("t.b") == b"b"


def _raw_shard(path, header: str, body: bytes, hlen=None):
    h = header.encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h) if hlen is None else hlen) + h + body)


BAD_CASES = {
    # name: (header, body, hlen override) -- rejected by both readers
    "span_mismatch": ('{"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 12]}}',
                      bytes(16), None),
    "past_eof": ('{"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}', bytes(8), None),
    "unknown_dtype": ('{"t": {"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}}',
                      bytes(8), None),
    "rank5": ('{"t": {"dtype": "U8", "shape": [1,1,1,1,1], "data_offsets": [0, 1]}}',
              bytes(1), None),
    "no_offsets": ('{"t": {"dtype": "U8", "shape": [1]}}', bytes(1), None),
    "no_dtype": ('{"t": {"shape": [1], "data_offsets": [0, 1]}}', bytes(1), None),
    "not_object": ('["t"]', b"", None),
    "hlen_impossible": ('{"t": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}',
                        bytes(1), 1 << 40),
    "hlen_zero": ("", bytes(8), 0),
    "bad_name": ('{t: {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', bytes(1), None),
}


@pytest.mark.parametrize("case", sorted(BAD_CASES))
def test_malformed_shards_rejected(gl, tmp_path, case):
    header, body, hlen = BAD_CASES[case]
    d = tmp_path / case
    d.mkdir()
    _raw_shard(str(d / "m.safetensors"), header, body, hlen)
    with pytest.raises(RuntimeError, match="dsv4g_st_open"):
        Checkpoint(str(d), gl)
    ref = ref_st(str(d))
    if ref is not None:
        assert not ref.ok, f"the reference reader accepts {case}"


def test_truncated_duplicate_and_empty(gl, tmp_path):
    d = tmp_path / "short"
    d.mkdir()
    (d / "m.safetensors").write_bytes(b"\x05\x00")
    with pytest.raises(RuntimeError, match="too short"):
        Checkpoint(str(d), gl)
    d = tmp_path / "dup"
    d.mkdir()
    write_safetensors(str(d / "a.safetensors"), [("same", "U8", (1,), b"a")])
    write_safetensors(str(d / "b.safetensors"), [("same", "U8", (1,), b"b")])
    with pytest.raises(RuntimeError, match="duplicate tensor name same"):
        Checkpoint(str(d), gl)
    ref = ref_st(str(d))
    if ref is not None:
        assert not ref.ok
    d = tmp_path / "empty"
    d.mkdir()
    with pytest.raises(RuntimeError, match="no .safetensors"):
        Checkpoint(str(d), gl)
    with pytest.raises(RuntimeError, match="cannot open directory"):
        Checkpoint(str(tmp_path / "absent"), gl)


def test_stricter_than_reference(gl, tmp_path):
    """Negative offsets or dimensions are refused here (the reference's
    integer parser accepts a sign)."""
    for i, hdr in enumerate(['{"t": {"dtype": "U8", "shape": [-1], "data_offsets": [1, 0]}}',
                             '{"t": {"dtype": "U8", "shape": [0], "data_offsets": [-4, -4]}}']):
        d = tmp_path / f"neg{i}"
        d.mkdir()
        _raw_shard(str(d / "m.safetensors"), hdr, bytes(4))
        with pytest.raises(RuntimeError):
            Checkpoint(str(d), gl)


def test_read_range_and_layer_bytes(gl, tmp_path):
    """dsv4g_st_read_range bounds, and the arena size of a layer: 256-byte
    aligned pieces in the order experts, gate, bias/tid2eid, sh1, sh1_s, sh3,
    sh3_s, sh2, sh2_s."""
    import ctypes as C
    from dsv4_gpu import DSV4GLayer
    ck = Checkpoint(ST_DIR, gl)
    buf = C.create_string_buffer(64)
    assert gl.lib.dsv4g_st_read_range(ck.h, 5, 0, 8, buf) == 0
    assert "bad shard" in gl.lib.dsv4g_last_error().decode()
    assert gl.lib.dsv4g_st_read_range(ck.h, 1, 0, 8, buf) == 8
    with open(ck.shard_path(1), "rb") as f:
        assert buf.raw[:8] == f.read(8)
    assert gl.lib.dsv4g_st_read_range(ck.h, 1, 970, 8, buf) == 3  # short at EOF

    def arena(H, I, E, K, is_hash, vocab):
        L = DSV4GLayer()
        L.hidden, L.inter, L.n_experts, L.topk = H, I, E, K
        return int(gl.lib.dsv4g_moe_layer_bytes(C.byref(L), is_hash, vocab))

    def al(v):
        return (v + 255) // 256 * 256

    H, I, E, K = 4096, 2048, 256, 6
    slot = 13369344
    sh = al(I * H) * 2 + al(H * I) + 3 * al(16 * 32)
    assert arena(H, I, E, K, 0, 0) == E * slot + al(E * H * 2) + al(E * 4) + sh
    assert arena(H, I, E, K, 1, 129280) == E * slot + al(E * H * 2) + al(129280 * K * 8) + sh
    assert arena(H, I, E, 0, 0, 0) == 0
    assert arena(H, I, E, K, 1, 0) == 0
