"""Device loads of safetensors tensors and the ANE blob writer
(core/safetensors.cpp:266-297, :316-383) on the GPU against the oracle:
loads are bit-exact (copy, exact widening, truncating convert); blob trees
are byte-identical to the oracle's, file by file."""
import os

import numpy as np
import pytest

from helpers import assert_bitexact, host

pytestmark = pytest.mark.gpu


def make_model(path, rng, big=20_000_003):
    import torch
    from safetensors.torch import save_file

    pats = torch.from_numpy(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16)).view(torch.bfloat16)
    ts = {
        "model.all_patterns.weight": pats.reshape(256, 256).contiguous(),
        "model.layers.0.mlp.gate_proj.weight": torch.randn(big).bfloat16(),       # spans 2 staging chunks
        "model.layers.0.self_attn.q_proj.weight": torch.randn(96, 64).bfloat16(),
        "model.layers.1.input_layernorm.weight": torch.randn(64).half(),            # not BF16: no blob
        "model.norm.weight": torch.randn(64),                                        # not BF16: no blob
        "lm_head.weight": torch.randn(1).bfloat16(),
        "model.empty.weight": torch.zeros(0).bfloat16(),
    }
    save_file(ts, str(path))
    return ts


def test_device_loads(hip, orc, tmp_path, rng):
    import torch

    p = tmp_path / "m.safetensors"
    make_model(p, rng)
    ref = orc.read_safetensors(str(p))
    with hip.SafeTensorsFile(p) as f:
        for name, (dt, shape, data) in ref.items():
            i = f.find(name)
            n = data.size
            if dt == "BF16":
                out32 = torch.empty(max(n, 1), device="cuda")
                f.load(i, out32, hip.F32)
                assert_bitexact(host(out32)[:n], orc.bf16_to_f32(data), name + " as f32")
                f.load_norm(i, out32, n)
                assert_bitexact(host(out32)[:n], orc.norm_weight(data), name + " as (1+w) norm weight")
                f.load_norm(i, out32, 0)                        # count <= 0: no offset, as the reference
                assert_bitexact(host(out32)[:n], orc.bf16_to_f32(data), name + " norm weight, count 0")
                if n:
                    with pytest.raises(hip.AnelmError, match="shape mismatch"):
                        f.load_norm(i, out32, n + 1)
                out16 = torch.empty(max(n, 1), dtype=torch.int16, device="cuda")
                f.load(i, out16, hip.F16)
                assert_bitexact(host(out16)[:n], orc.bf16_to_f16(data), name + " as f16")
                raw = torch.empty(max(n, 1), dtype=torch.int16, device="cuda")
                f.load(i, raw, hip.BF16)
                assert_bitexact(host(raw)[:n], data, name + " raw")
            elif dt == "F32":
                out = torch.empty(n, device="cuda")
                f.load(i, out, hip.F32)
                assert_bitexact(host(out), data, name)
                with pytest.raises(hip.AnelmError):
                    f.load(i, out, hip.F16)                     # only BF16 converts
                with pytest.raises(hip.AnelmError, match="not BF16"):
                    f.load_norm(i, out, n)


def _tree(root):
    files = {}
    for d, _, names in os.walk(root):
        for n in names:
            full = os.path.join(d, n)
            files[os.path.relpath(full, root)] = open(full, "rb").read()
    return files


def test_write_ane_blobs_byte_identical(hip, orc, tmp_path, rng):
    p = tmp_path / "m.safetensors"
    make_model(p, rng)
    got_dir, ref_dir = tmp_path / "got", tmp_path / "ref"
    n = hip.write_ane_blobs(p, got_dir)
    m = orc.write_ane_blobs(str(p), str(ref_dir))
    assert n == m == 5
    got, ref = _tree(got_dir), _tree(ref_dir)
    assert sorted(got) == sorted(ref)
    for k in ref:
        assert got[k] == ref[k], k
    assert len(got["model/empty/weight.bin"]) == 128


def test_write_ane_blobs_errors(hip, tmp_path):
    with pytest.raises(hip.AnelmError):
        hip.write_ane_blobs(tmp_path / "absent.safetensors", tmp_path / "out")
