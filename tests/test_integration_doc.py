"""The integration guide's documented calls compile against the library's headers
(include/anelm_hip.h and the ane_lm:: drop-in headers), and the check
catches a wrong argument order.  CPU only: g++ -fsyntax-only."""
import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp"))
import integration_doc  # noqa: E402


def test_every_documented_call_compiles(tmp_path):
    blocks, calls = integration_doc.extract(open(integration_doc.DOC, encoding="utf-8").read())
    assert len(blocks) >= 6 and len(calls) >= 3
    assert any("qknorm_rope_qwen3" in c for c in calls)
    integration_doc.check(out_dir=str(tmp_path))


@pytest.mark.parametrize("good,bad", [
    # the drop-in q/k norm + RoPE with the position before the gammas
    ("lw.q_norm, lw.k_norm, eps, pos, theta,", "pos, theta, lw.q_norm, lw.k_norm, eps,"),
    # the attention's ring state and caches swapped
    ("k_cache[L], v_cache[L], kv_start[L], kv_len[L], B, nq, nk, 128,",
     "kv_start[L], kv_len[L], k_cache[L], v_cache[L], B, nq, nk, 128,"),
    # an argument dropped from the fused projection
    ("anelm_proj_f16_x16_fused(x, h16, lw.Wdown, B, H, I, I, H, ANELM_PROJ_ADD, s);",
     "anelm_proj_f16_x16_fused(x, h16, lw.Wdown, B, H, I, I, ANELM_PROJ_ADD, s);"),
    # an argument dropped from the tiled projection
    ("anelm_proj_f16_tt(x, h16, lw.Wdown_t, B, H, I, H, ANELM_PROJ_ADD, s);",
     "anelm_proj_f16_tt(x, h16, lw.Wdown_t, B, H, I, ANELM_PROJ_ADD, s);"),
])
def test_planted_mistake_fails(tmp_path, good, bad):
    md = open(integration_doc.DOC, encoding="utf-8").read()
    assert good in md
    with pytest.raises(RuntimeError):
        integration_doc.check(md.replace(good, bad, 1), out_dir=str(tmp_path))
