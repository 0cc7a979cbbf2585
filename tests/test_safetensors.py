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


_SIZES = {"BF16": 2, "F16": 2, "F32": 4, "F64": 8, "I32": 4, "I64": 8, "U8": 1}


def _check_open(path):
    """Open a possibly malformed file: either an AnelmError, or a handle whose
    every tensor lies inside the data block with bytes = numel x dtype size."""
    import anelm

    raw = path.read_bytes()
    try:
        f = anelm.SafeTensorsFile(path)
    except anelm.AnelmError:
        return False
    with f:
        hlen = struct.unpack("<Q", raw[:8])[0]
        data = len(raw) - 8 - hlen
        assert data >= 0
        for i in range(len(f)):
            name, dt, shape, off, nb = f.info(i)
            assert off + nb <= data, (name, off, nb, data)
            assert all(d >= 0 for d in shape)
            size = {anelm.BF16: 2, anelm.F16: 2, anelm.F32: 4, anelm.ST_F64: 8, anelm.ST_I32: 4, anelm.ST_I64: 8,
                    anelm.ST_U8: 1}.get(dt)
            if size is not None:
                assert int(np.prod(shape, dtype=np.int64)) * size == nb, (name, shape, nb)
    return True


def test_fuzz_mutated_and_truncated_files(tmp_path, rng):
    """Byte mutations inside the header, length-field changes and
    truncations of a valid file never crash the parser, and whatever it
    accepts is consistent (no tensor outside the data block)."""
    p = tmp_path / "m.safetensors"
    make_file(p, rng)
    good = p.read_bytes()
    hlen = struct.unpack("<Q", good[:8])[0]
    q = tmp_path / "fuzz.safetensors"
    accepted = 0
    for trial in range(400):
        b = bytearray(good)
        kind = trial % 4
        if kind == 0:      # flip bytes inside the JSON header
            for _ in range(int(rng.integers(1, 4))):
                b[8 + int(rng.integers(0, hlen))] = int(rng.integers(0, 256))
        elif kind == 1:    # digits changed: offsets and shapes
            digits = [i for i in range(8, 8 + hlen) if chr(b[i]).isdigit()]
            for _ in range(int(rng.integers(1, 3))):
                b[digits[int(rng.integers(0, len(digits)))]] = ord(str(int(rng.integers(0, 10))))
        elif kind == 2:    # the header length field
            b[:8] = struct.pack("<Q", int(rng.integers(0, len(good) + 64)))
        else:              # truncation
            b = b[:int(rng.integers(0, len(good)))]
        q.write_bytes(bytes(b))
        accepted += _check_open(q)
    assert accepted > 0   # some mutations (e.g. inside names) stay valid


@pytest.mark.parametrize("seed", range(6))
def test_fuzz_random_headers(tmp_path, seed):
    """Structured random headers: unknown dtypes, negative, zero and huge
    dimensions, offsets out of order, overlapping or past the end, odd
    metadata."""
    r = np.random.default_rng(100 + seed)
    q = tmp_path / "h.safetensors"
    for _ in range(60):
        hdr = {}
        for t in range(int(r.integers(0, 5))):
            dt = str(r.choice(["BF16", "F16", "F32", "F64", "I32", "I64", "U8", "BOOL", "F8_E4M3", ""]))
            shape = [int(x) for x in r.choice([0, 1, 3, 4, -1, 1 << 31, 1 << 62], int(r.integers(0, 4)))]
            a = int(r.choice([0, 4, 8, 16, 1 << 40, -8]))
            b = a + int(r.choice([0, 2, 8, 24, -2]))
            hdr[f"t{t}"] = {"dtype": dt, "shape": shape, "data_offsets": [a, b]}
        if r.random() < 0.3:
            hdr["__metadata__"] = {"k": str(r.integers(0, 9))}
        _write_raw(q, hdr, bytes(int(r.integers(0, 64))))
        _check_open(q)
