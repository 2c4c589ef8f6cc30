"""Safetensors reading in libq35mm.so (q35mm_st_*), on the CPU: no GPU call
is made by opening, indexing or reading a checkpoint.

Checks follow the reference's reader and its test (qwen35-c/src/q35_st.c,
qwen35-c/tests/test_st.c): its mini.safetensors fixture (names, dtypes,
shapes, CRC-32 of the bytes from its manifest), a header truncated to 64
bytes, and synthetic files for each validation rule (header length bounds,
malformed JSON, unknown dtype, offsets out of the file, byte counts that do
not match the shape), shard directories and the shard-name rule.
"""
import json
import os
import struct
import zlib

import numpy as np
import pytest

from conftest import GOLDEN

ST = os.path.join(GOLDEN, "st")
EIO, EFORMAT, ENOTFOUND = -5, -6, -7


def write_st(path, tensors, meta=None, header_pad=0, raw_header=None):
    """tensors: list of (name, dtype, shape, bytes)."""
    hdr, blobs, off = {}, [], 0
    if meta is not None:
        hdr["__metadata__"] = meta
    for name, dt, shape, data in tensors:
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    h = raw_header if raw_header is not None else json.dumps(hdr).encode() + b" " * header_pad
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)
    return path


def code_of(excinfo):
    return getattr(excinfo.value, "code", None)


def test_reference_mini_fixture(q):
    ck = q.Checkpoint(os.path.join(ST, "mini.safetensors"))
    man = [ln.split() for ln in open(os.path.join(ST, "mini_manifest.txt")) if ln.strip()]
    assert sorted(ck.names()) == sorted(m[0] for m in man)
    for name, shape, dtype, crc in man:
        dt, shp, nb = ck.info(name)
        assert dt == dtype
        assert shp == tuple(int(v) for v in shape.split("x"))
        data = ck.read(name)
        assert len(data) == nb
        assert "%08x" % (zlib.crc32(data) & 0xFFFFFFFF) == crc
    with pytest.raises(q.Q35mmError) as e:
        ck.info("does.not.exist")
    assert code_of(e) == ENOTFOUND
    ck.close()


def test_truncated_header_is_rejected(q, tmp_path):
    head = open(os.path.join(ST, "mini.safetensors"), "rb").read(64)
    p = tmp_path / "trunc.safetensors"
    p.write_bytes(head)
    with pytest.raises(q.Q35mmError) as e:
        q.Checkpoint(str(p))
    assert code_of(e) == EFORMAT


def test_reference_model_checkpoint_index(q):
    ck = q.Checkpoint(os.path.join(ST, "model.safetensors"))
    names = ck.names()
    assert "lm_head.weight" in names
    fp8 = [n for n in names if ck.info(n)[0] == "F8_E4M3"]
    assert len(fp8) >= 20
    for n in fp8:
        dt, (rows, cols), nb = ck.info(n)
        sdt, sshape, _ = ck.info(n + "_scale_inv")
        assert nb == rows * cols
        assert sdt == "BF16" and sshape == ((rows + 127) // 128, (cols + 127) // 128)


@pytest.mark.parametrize("case", ["zero_len", "huge_len", "bad_json", "not_object", "bad_dtype", "past_end",
                                  "wrong_size", "reversed", "shape_not_int", "nine_dims", "header_past_file"])
def test_header_validation(q, tmp_path, case):
    p = str(tmp_path / "x.safetensors")
    good = [("w", "F32", (2, 3), np.arange(6, dtype=np.float32).tobytes())]
    want = EFORMAT
    if case == "zero_len":
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", 0))
    elif case == "huge_len":
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", (1 << 24) + 1) + b"{}")
    elif case == "bad_json":
        write_st(p, good, raw_header=b'{"w": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]}')
    elif case == "not_object":
        write_st(p, good, raw_header=b'[1, 2]')
    elif case == "bad_dtype":
        write_st(p, [("w", "U8", (6,), bytes(6))])
    elif case == "past_end":
        write_st(p, good, raw_header=json.dumps({"w": {"dtype": "F32", "shape": [2, 3],
                                                       "data_offsets": [0, 1000]}}).encode())
    elif case == "wrong_size":
        write_st(p, good, raw_header=json.dumps({"w": {"dtype": "F32", "shape": [2, 4],
                                                       "data_offsets": [0, 24]}}).encode())
    elif case == "reversed":
        write_st(p, good, raw_header=json.dumps({"w": {"dtype": "F32", "shape": [0],
                                                       "data_offsets": [24, 0]}}).encode())
    elif case == "shape_not_int":
        write_st(p, good, raw_header=json.dumps({"w": {"dtype": "F32", "shape": [2, 3.5],
                                                       "data_offsets": [0, 24]}}).encode())
    elif case == "nine_dims":
        write_st(p, [("w", "F32", (1,) * 9, bytes(4))])
    elif case == "header_past_file":
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", 100) + b'{"a": 1}')
    with pytest.raises(q.Q35mmError) as e:
        q.Checkpoint(p)
    assert code_of(e) == want, str(e.value)


def test_missing_file_and_empty_directory(q, tmp_path):
    with pytest.raises(q.Q35mmError) as e:
        q.Checkpoint(str(tmp_path / "nope.safetensors"))
    assert code_of(e) == EIO
    (tmp_path / "config.json").write_text("{}")
    with pytest.raises(q.Q35mmError) as e:
        q.Checkpoint(str(tmp_path))
    assert code_of(e) == EIO


def test_metadata_escapes_padding_and_empty_tensors(q, tmp_path):
    p = str(tmp_path / "m.safetensors")
    a = np.arange(12, dtype=np.float32)
    name = 'odd \\"name\\" \\u00e9\\ud83d\\ude00/x'
    hdr = ('{"__metadata__": {"format": "pt", "note": "x"}, "%s": {"dtype": "F32", "shape": [3, 4], '
           '"data_offsets": [0, 48]}, "empty": {"dtype": "BF16", "shape": [0, 5], "data_offsets": [48, 48]}, '
           '"s": {"dtype": "I64", "shape": [], "data_offsets": [48, 56]}}' % name).encode() + b"        "
    write_st(p, [("x", "F32", (12,), a.tobytes() + struct.pack("<q", -7))], raw_header=hdr)
    ck = q.Checkpoint(p)
    decoded = 'odd "name" é\U0001F600/x'
    assert sorted(ck.names()) == sorted([decoded, "empty", "s"])
    dt, shape, nb = ck.info(decoded)
    assert dt == "F32" and shape == (3, 4) and nb == 48
    assert np.frombuffer(ck.read(decoded), np.float32).tolist() == a.tolist()
    assert ck.info("empty") == ("BF16", (0, 5), 0)
    assert ck.info("s") == ("I64", (), 8)
    assert struct.unpack("<q", ck.read("s"))[0] == -7


def test_shard_directory(q, tmp_path):
    d = tmp_path / "ckpt"
    d.mkdir()
    x = np.arange(8, dtype=np.float32)
    write_st(str(d / "model-00001-of-00002.safetensors"), [("a", "F32", (8,), x.tobytes())])
    write_st(str(d / "model-00002-of-00002.safetensors"), [("b", "BF16", (2, 2), bytes(range(8)))])
    (d / "model.safetensors.index.json").write_text('{"weight_map": {}}')   # not a shard
    (d / "config.json").write_text("{}")
    ck = q.Checkpoint(str(d))
    assert sorted(ck.names()) == ["a", "b"]
    assert ck.read("b") == bytes(range(8))
    assert np.frombuffer(ck.read("a"), np.float32).tolist() == x.tolist()
    # a bad shard fails the whole directory, as the reference's reader does
    (d / "zz.safetensors").write_bytes(b"\x00" * 4)
    with pytest.raises(q.Q35mmError) as e:
        q.Checkpoint(str(d))
    assert code_of(e) == EFORMAT
