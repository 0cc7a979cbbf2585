"""The safetensors reader (core/safetensors.cpp:58-253) and the ANE blob
header (core/safetensors.cpp:316-331) on the CPU: the oracle reader is
pinned against the safetensors package (the format's own implementation),
the library's parser against the oracle reader, and the header against the
reference's literal byte layout.  No GPU calls."""
import json
import os
import struct

import numpy as np
import pytest


def make_file(path, rng):
    import torch
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(3)
    ts = {
        "model.embed_tokens.weight": torch.randn(64, 16, generator=g).bfloat16(),
        "model.layers.0.self_attn.q_proj.weight": torch.randn(32, 16, generator=g).bfloat16(),
        "model.layers.0.input_layernorm.weight": torch.randn(16, generator=g).half(),
        "model.layers.0.mlp.scale": torch.randn(3, 5, generator=g),
        "model.layers.0.counts": torch.arange(7, dtype=torch.int64),
        "lm_head.weight": torch.randn(1, generator=g).bfloat16(),
        "empty.weight": torch.zeros(0, 4).bfloat16(),
        "bytes": torch.arange(10, dtype=torch.uint8),
    }
    save_file(ts, str(path), metadata={"format": "pt", "note": "a {brace} and \"quotes\""})
    return ts


def test_oracle_reader_matches_safetensors_package(orc, tmp_path, rng):
    import torch

    p = tmp_path / "m.safetensors"
    ts = make_file(p, rng)
    got = orc.read_safetensors(str(p))
    assert set(got) == set(ts)
    for name, t in ts.items():
        dt, shape, data = got[name]
        assert shape == tuple(t.shape)
        want = t.view(torch.int16).numpy().view(np.uint16) if t.dtype in (torch.bfloat16, torch.float16) else t.numpy()
        assert np.array_equal(data, want.ravel()), name
        assert dt == {torch.bfloat16: "BF16", torch.float16: "F16", torch.float32: "F32", torch.int64: "I64",
                      torch.uint8: "U8"}[t.dtype]


def test_library_parser_matches_oracle(orc, tmp_path, rng):
    import anelm

    p = tmp_path / "m.safetensors"
    make_file(p, rng)
    ref = orc.read_safetensors(str(p))
    raw = p.read_bytes()
    hlen = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + hlen])
    codes = {"BF16": anelm.BF16, "F16": anelm.F16, "F32": anelm.F32, "I64": anelm.ST_I64, "U8": anelm.ST_U8}
    with anelm.SafeTensorsFile(p) as f:
        assert len(f) == len(ref)
        names = [f.info(i)[0] for i in range(len(f))]
        assert set(names) == set(ref)
        for i, name in enumerate(names):
            n, dt, shape, off, nb = f.info(i)
            a, b = header[name]["data_offsets"]
            assert (dt, shape, off, nb) == (codes[ref[name][0]], ref[name][1], a, b - a)
            assert f.find(name) == i
            if nb:
                import ctypes
                data = ctypes.string_at(f.host_data(i), nb)
                assert data == ref[name][2].tobytes()
        assert f.find("no.such.tensor") == -1


def _write_raw(path, header: dict, data: bytes):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)


@pytest.mark.parametrize("case", ["offsets_beyond_file", "shape_mismatch", "header_too_long", "not_json", "missing"])
def test_malformed_files_are_errors(tmp_path, case):
    import anelm

    p = tmp_path / "bad.safetensors"
    if case == "offsets_beyond_file":
        _write_raw(p, {"w": {"dtype": "BF16", "shape": [4], "data_offsets": [0, 8]}}, b"\0" * 4)
    elif case == "shape_mismatch":
        _write_raw(p, {"w": {"dtype": "BF16", "shape": [5], "data_offsets": [0, 8]}}, b"\0" * 8)
    elif case == "header_too_long":
        p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    elif case == "not_json":
        p.write_bytes(struct.pack("<Q", 5) + b"{nope")
    else:
        p = tmp_path / "absent.safetensors"
    with pytest.raises(anelm.AnelmError) as e:
        anelm.SafeTensorsFile(p)
    assert e.value.args


@pytest.mark.parametrize("n", [0, 1, 7, 1 << 20, (1 << 31) + 3])
def test_blob_header_layout(orc, n):
    """Bytes 0 = 1, 4 = 2; chunk header at 64: EF BE AD DE, version 1, the
    fp16 data size (u32, the reference's truncating cast) and offset 128."""
    import anelm

    h = anelm.ane_blob_header(n)
    assert len(h) == 128
    want = bytearray(128)
    want[0], want[4] = 1, 2
    want[64:68] = b"\xef\xbe\xad\xde"
    want[68] = 1
    want[72:76] = struct.pack("<I", (2 * n) & 0xFFFFFFFF)
    want[80:84] = struct.pack("<I", 128)
    assert h == bytes(want)
    if n < (1 << 21):
        assert orc.ane_blob(np.zeros(n, np.uint16))[:128] == h


def test_blob_paths(orc):
    assert orc.blob_relpath("model.layers.0.mlp.gate_proj.weight") == "model/layers/0/mlp/gate_proj/weight.bin"
