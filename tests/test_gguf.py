"""GGUF loader (okf_gguf_*): parsing, metadata, directory and errors, on
synthetic files written by tests/ggufw.py.  CPU only (no device calls)."""
import numpy as np
import pytest

import chatokf_amd as ok
from chatokf_amd import synth
from chatokf_amd.formats import Q8_0, Q4_K, row_bytes

import ggufw as gw


def make(tmp_path, **kw):
    q4 = synth.q4_k(3, 512, 5).tobytes()
    q8 = synth.q8_0(2, 64, 6).tobytes()
    f32 = np.arange(4, dtype=np.float32).tobytes()
    kvs = [("general.architecture", gw.STR, "qwen35"), ("general.alignment", gw.U32, 64),
           ("n.u8", gw.U8, 200), ("n.i32", gw.I32, -7), ("n.u64", gw.U64, 1 << 40),
           ("x.f32", gw.F32, 0.5), ("x.f64", gw.F64, -2.25), ("flag", gw.BOOL, 1),
           ("tok.list", gw.ARR, (gw.STR, ["a", "bc", ""])), ("ints", gw.ARR, (gw.I32, [1, -2, 3]))]
    tensors = [("blk.0.ffn_down.weight", [512, 3], Q4_K, q4), ("tiny", [64, 2], Q8_0, q8),
               ("norm", [4], 0, f32)]
    path = tmp_path / "t.gguf"
    offs, data_start = gw.write(path, kvs, tensors, alignment=64, **kw)
    return path, tensors, offs, data_start


def test_directory_metadata_and_data(tmp_path):
    path, tensors, offs, data_start = make(tmp_path)
    with ok.GGUF(str(path)) as g:
        ts = g.tensors()
        assert [t["name"] for t in ts] == [t[0] for t in tensors]
        assert [t["dims"] for t in ts] == [t[1] for t in tensors]
        assert [t["type"] for t in ts] == [t[2] for t in tensors]
        assert [t["offset"] for t in ts] == offs
        assert [t["bytes"] for t in ts] == [row_bytes(Q4_K, 1536), row_bytes(Q8_0, 128), 16]
        blob = g.data()
        raw = path.read_bytes()
        assert blob == raw[data_start:]
        for t, (_, _, _, data) in zip(ts, tensors):
            assert blob[t["offset"]:t["offset"] + t["bytes"]] == data
        assert g.string("general.architecture") == "qwen35"
        assert g.int("general.alignment") == 64
        assert g.int("n.u8") == 200 and g.int("n.i32") == -7 and g.int("n.u64") == 1 << 40
        assert g.double("x.f32") == 0.5 and g.double("x.f64") == -2.25
        assert g.double("n.i32") == -7.0           # GGUF.double reads ints too
        assert g.int("flag") == 1                  # a bool reads as 0 / 1
        assert g.int("missing") is None and g.string("n.u8") is None
        assert g.find("nope") is None
        w = g.weight("blk.0.ffn_down.weight", 0x1000)
        assert (w.K, w.M, w.type, w.off) == (512, 3, Q4_K, offs[0])


@pytest.mark.parametrize("kw,status", [
    ({"magic": b"GGUX"}, ok.OKF_E_FORMAT),
    ({"truncate": 40}, ok.OKF_E_FORMAT),     # inside the key/values
    ({"truncate": 900}, ok.OKF_E_FORMAT),    # a tensor past the end of the file
])
def test_malformed_files_are_rejected(tmp_path, kw, status):
    path, *_ = make(tmp_path, **kw)
    with pytest.raises(ok.OkfError) as e:
        ok.GGUF(str(path))
    assert e.value.status == status


def test_unknown_type_and_missing_file(tmp_path):
    path = tmp_path / "u.gguf"
    gw.write(path, [], [("w", [32, 1], 99, b"\0" * 64)])
    with pytest.raises(ok.OkfError) as e:
        ok.GGUF(str(path))
    assert e.value.status == ok.OKF_E_FORMAT
    with pytest.raises(ok.OkfError) as e:
        ok.GGUF(str(tmp_path / "absent.gguf"))
    assert e.value.status == ok.OKF_E_IO


def test_upload_needs_a_device(tmp_path):
    path, *_ = make(tmp_path)
    e = ok.Enc(-1)
    with ok.GGUF(str(path)) as g, pytest.raises(ok.OkfError) as err:
        g.upload(e)
    assert err.value.status == ok.OKF_E_NODEV
    e.close()


def test_tensorless_file_ending_before_the_alignment(tmp_path):
    # no tensors, and the directory ends inside the last alignment unit: the
    # data region would start past the end of the file
    path = tmp_path / "e.gguf"
    gw.write(path, [("general.alignment", gw.U32, 256)], [])
    raw = path.read_bytes()
    path.write_bytes(raw[:len(raw) - 100])  # drop part of the trailing padding
    with pytest.raises(ok.OkfError) as e:
        ok.GGUF(str(path))
    assert e.value.status == ok.OKF_E_FORMAT


@pytest.mark.parametrize("dims", [[1 << 32, 1 << 32, 1 << 8], [1 << 62, 4], [(1 << 64) - 1, 2]])
def test_overflowing_dims_are_rejected(tmp_path, dims):
    # element counts whose product (or byte count) would wrap to a small value
    path = tmp_path / "o.gguf"
    gw.write(path, [], [("w", dims, 0, b"\0" * 64)])
    with pytest.raises(ok.OkfError) as e:
        ok.GGUF(str(path))
    assert e.value.status == ok.OKF_E_FORMAT


@pytest.mark.parametrize("alignment", [0, 48, 1 << 21])
def test_bad_alignment_is_rejected(tmp_path, alignment):
    path = tmp_path / "a.gguf"
    gw.write(path, [("general.alignment", gw.U32, alignment)], [("w", [32, 1], 0, b"\0" * 128)])
    with pytest.raises(ok.OkfError) as e:
        ok.GGUF(str(path))
    assert e.value.status == ok.OKF_E_FORMAT
