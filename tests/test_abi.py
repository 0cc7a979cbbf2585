"""The C-ABI library loads and exports every symbol include/anelm_hip.h
declares, plus the ane_lm:: drop-in functions; argument validation fails
with a status and a message before anything touches the GPU.  No compute
calls: this runs without a GPU."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "anelm_hip.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(anelm_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    import anelm

    return anelm.lib()


def test_header_declares_the_path():
    names = declared()
    for n in ["anelm_rmsnorm", "anelm_add_rmsnorm", "anelm_qknorm_rope", "anelm_rope_cached", "anelm_rope_table",
              "anelm_residual_add", "anelm_silu_mul", "anelm_silu", "anelm_mul_sigmoid", "anelm_embed_gather",
              "anelm_bf16_to_f16", "anelm_softmax", "anelm_sample", "anelm_sample_workspace_size",
              "anelm_last_error"]:
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    import anelm

    assert sorted(anelm.EXPORTED) == declared()


def test_dropin_cpp_symbols_exported():
    import anelm

    out = subprocess.run(["nm", "-D", "--defined-only", "-C", anelm.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    for sig in ["ane_lm::rmsnorm(float*, float const*, float const*, int, float)",
                "ane_lm::softmax(float*, int)",
                "ane_lm::silu_vec_inplace(float*, int, float*)",
                "ane_lm::mul_sigmoid_inplace(float*, float const*, int, float*)",
                "ane_lm::apply_rope_cached(float*, float*, int, int, int, int, int, int, int, float, float const*, float const*)",
                "ane_lm::sample_token(float const*, int, ane_lm::SamplingParams const&, std::vector<int, std::allocator<int> > const&)",
                "ane_lm::hip::bf16_to_f16_vec(unsigned short*, unsigned short const*, int)",
                "ane_lm::hip::residual_add(float*, float const*, int)",
                "ane_lm::gqa_attention(float*, float const*, float const*, float const*, int, int, int, int, int, int, int)",
                "ane_lm::rmsnorm_gated(float*, float const*, float const*, float const*, int)",
                "ane_lm::matvec(float*, float const*, float const*, int, int)",
                "ane_lm::l2_normalize(float*, int)",
                "ane_lm::conv1d_update(float*, float*, int*, float const*, float const*, int, int)",
                "ane_lm::ssm_step(float*, float*, float const*, float const*, float const*, float, float, int, int)"]:
        assert sig in out, sig


def test_version(lib):
    assert lib.anelm_version() >= 100


def test_invalid_arguments_return_status_and_message(lib):
    P = ctypes.c_void_p
    assert lib.anelm_rmsnorm(None, None, None, 0, 1, 16, 16, 16, 1e-6, None) == -1
    assert b"null" in lib.anelm_last_error()
    fake = P(0x1000)  # never dereferenced: validation fails first
    assert lib.anelm_rmsnorm(fake, fake, fake, 0, 0, 16, 16, 16, 1e-6, None) == -1
    assert lib.anelm_rmsnorm(fake, fake, fake, 0, 4, 16, 8, 16, 1e-6, None) == -1       # ld < dim
    assert lib.anelm_rmsnorm(fake, fake, fake, 7, 4, 16, 16, 16, 1e-6, None) == -1      # dtype
    assert lib.anelm_add_rmsnorm(fake, fake, fake, fake, 0, 4, 16, 16, 16, 16, 1e-6, None) == -1  # out == x
    assert lib.anelm_qknorm_rope(fake, fake, 128, 128, None, None, 0, None, None, None, 0, 1e6, 1, 1, 1, 128,
                                 1e-6, None) == -1                                       # null pos
    assert lib.anelm_qknorm_rope(fake, fake, 128, 128, None, None, 0, fake, None, None, 0, 1e6, 1, 1, 1, 127,
                                 1e-6, None) == -1                                       # odd head_dim
    assert lib.anelm_residual_add(fake, fake, 0, None) == -1
    assert lib.anelm_bf16_to_f16(None, fake, 8, None) == -1
    assert lib.anelm_embed_gather(fake, fake, 1, fake, 70000, 16, 16, None, None) == -1  # grid.y limit
    import anelm

    p = anelm.SamplingParams()
    assert lib.anelm_sample(fake, None, 0, fake, 100, 1, 100, None, 0, None, ctypes.byref(p), None, fake, 1 << 20,
                            None) == -1                                                  # r required
    assert lib.anelm_sample(fake, None, 0, fake, 100, 1, 100, None, 0, None, ctypes.byref(p), fake, fake, 1 << 20,
                            None) == -1                                                  # probs required
    assert lib.anelm_sample(fake, fake, 100, fake, 100, 1, 100, None, 0, None, ctypes.byref(p), fake, fake, 16,
                            None) == -4                                                  # workspace too small
    assert b"workspace" in lib.anelm_last_error()
    # tiled projection: in_dim not a multiple of 32, unknown epilogue, a SwiGLU whose gate rows are not a
    # multiple of 16, W overlapping its tiled copy
    lib.anelm_proj_tiled_size.restype = ctypes.c_size_t
    assert lib.anelm_proj_tiled_size(100, 1000) == 0
    assert lib.anelm_proj_tile_f16(fake, P(0x2000), 100, 1000, None) == -1
    assert lib.anelm_proj_tile_f16(fake, P(0x1100), 100, 1024, None) == -1             # overlap
    assert b"overlap" in lib.anelm_last_error()
    assert lib.anelm_proj_f16_x16_tiled(P(0x100000), P(0x200000), P(0x300000), 64, 1000, 200, 200, 1000, 0,
                                        None) == -1                                      # in_dim % 32
    assert lib.anelm_proj_f16_x16_tiled(P(0x100000), P(0x200000), P(0x300000), 64, 1000, 256, 256, 1000, 5,
                                        None) == -1                                      # no such epilogue
    assert b"epilogue" in lib.anelm_last_error()
    assert lib.anelm_proj_f16_x16_tiled(P(0x100000), P(0x200000), P(0x300000), 64, 1000, 256, 256, 1000, 2,
                                        None) == -1                                      # SwiGLU, 1000 % 16
    assert b"multiple of 16" in lib.anelm_last_error()


def test_tiled_size(lib):
    lib.anelm_proj_tiled_size.restype = ctypes.c_size_t
    # rows padded to a multiple of 16, fp16
    assert lib.anelm_proj_tiled_size(151936, 1024) == 151936 * 1024 * 2
    assert lib.anelm_proj_tiled_size(70001, 256) == 70016 * 256 * 2


def test_workspace_sizes(lib):
    # the one-launch path's epoch (256 bytes), its per-row tokens (two u64) and
    # its two barriers' flags (u64 per row and chunk of its smallest chunks,
    # 4096 logits: 38 at 151936), then 64 rows x 50 chunks of 3072 logits (u64 sums, f32 maxima,
    # i32 argmax, i32 flags) + 64 rows x 594 sub-tiles of 256, rows padded to
    # 596 (two u32 map words, i32 binade class, six u32 words of the predicted
    # crossing), 16-byte aligned
    al = lambda b: (b + 15) // 16 * 16
    tok = lambda rows: 256 + al(rows * 16) + al(rows * 2 * 38 * 8)
    n, ns = 64 * 50, 64 * 596
    assert lib.anelm_sample_workspace_size(64, 151936) == (tok(64) + al(n * 8) + 3 * al(n * 4) + 3 * al(ns * 4)
                                                           + al(ns * 24) + al(64 * 8))   # + sub-tile 0 result per row
    # fewer rows (rows x 149 chunks of 1024 < 3600 workgroups): chunks of 1024, 149 per row
    n, ns = 24 * 149, 24 * 596
    assert lib.anelm_sample_workspace_size(24, 151936) == (tok(24) + al(n * 8) + 3 * al(n * 4) + 3 * al(ns * 4)
                                                           + al(ns * 24) + al(24 * 8))
    n, ns = 25 * 50, 25 * 596
    assert lib.anelm_sample_workspace_size(25, 151936) == (tok(25) + al(n * 8) + 3 * al(n * 4) + 3 * al(ns * 4)
                                                           + al(ns * 24) + al(25 * 8))
    assert lib.anelm_sample_workspace_size(0, 10) == 0
    assert lib.anelm_softmax_workspace_size(1, 4096) > 0


def test_error_string_is_per_thread(lib):
    import threading

    lib.anelm_residual_add(None, None, 1, None)
    seen = {}

    def other():
        seen["msg"] = lib.anelm_last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == b""
    assert b"null" in lib.anelm_last_error()


def test_attention_argument_checks(lib):
    """Validation of the KV-ring / attention entry points (no launch happens)."""
    P = ctypes.c_void_p
    fake = P(0x1000)
    ws = lib.anelm_gqa_workspace_size
    # the chunk is 512 positions once there are >= 2048 workgroups, else it
    # shrinks towards 64; a call's partials (rounded up to 256 bytes) sit
    # below the counter region, the workspace's last 64th from a 256-byte
    # boundary, which holds one counter per (sequence, kv head).  The size
    # for a batch serves every smaller batch.
    up = lambda n: (n + 255) // 256 * 256

    def chunk(b, nkv, cap):
        for c in (512, 256, 128):
            if b * nkv * -(-cap // c) >= 2048:
                return c
        return 64

    def partials(b, nh, nkv, d, cap):
        ns = -(-cap // chunk(b, nkv, cap))
        return up(b * nh * ns * (d + 2) * 4) if ns > 1 else 0

    for B, nh, nkv, d, cap in ((64, 32, 8, 128, 2048), (1, 32, 8, 128, 2048), (3, 12, 4, 64, 1000),
                               (4, 32, 8, 128, 32768), (200, 16, 8, 128, 4096)):
        n = ws(B, nh, nkv, d, cap)
        region = (n - n // 64) & ~255
        assert max(partials(b, nh, nkv, d, cap) for b in range(1, B + 1)) <= region
        assert (n - region) // 4 >= B * nkv
        assert n <= 1.05 * max(partials(b, nh, nkv, d, cap) for b in range(1, B + 1)) + 1024   # about 1/63 more
    assert partials(3, 32, 8, 128, 32768) > partials(4, 32, 8, 128, 32768)   # a smaller batch needing more
    assert ws(512, 16, 8, 128, 512) > 0                         # one chunk at 512 sequences, not at fewer
    assert ws(4, 16, 8, 128, 64) == 0                           # one chunk at any batch: no partials
    assert ws(0, 32, 8, 128, 2048) == 0
    g = lib.anelm_gqa_attention
    ok = dict(q_ld=32 * 128, qs=128, out_ld=32 * 128, cap=2048, seq=2048 * 8 * 128)

    def call(nh=32, nkv=8, d=128, ring=fake, batch=2, ws_bytes=1 << 30, **kw):
        a = dict(ok, **kw)
        return g(fake, fake, fake, fake, ring, ring, batch, nh, nkv, d, a["q_ld"], a["qs"], a["out_ld"], a["cap"],
                 a["seq"], fake, ws_bytes, None)

    assert call(d=96) == -1 and b"head_dim" in lib.anelm_last_error()
    assert call(nh=30) == -1                                    # not a multiple of n_kv_heads
    assert call(ring=None) == -1
    assert call(seq=100) == -1                                  # sequences' caches overlap
    assert call(qs=130) == -1                                   # stride not a multiple of 4
    assert call(ws_bytes=16) == -4                              # workspace too small
    r = lib.anelm_gqa_attention_ring
    assert r(fake, fake, fake, fake, 32, 8, 128, 128, 0, 2049, 2048, fake, 1 << 30, None) == -2  # len > capacity
    assert r(fake, fake, fake, fake, 32, 8, 128, 128, 2048, 5, 2048, fake, 1 << 30, None) == -2  # start outside
    assert r(fake, fake, fake, fake, 32, 8, 128, 128, -1, 5, 2048, fake, 1 << 30, None) == -2
    qk = lib.anelm_gqa_attention_qk

    def call_qk(wq=fake, tab_len=4096, k_ld=48 * 128, batch=2, dt=2):
        row = 48 * 128
        return qk(fake, 1, fake, fake, fake, row, k_ld, row, wq, fake, dt, fake, fake, fake, tab_len, 1e6, 1e-6, fake,
                  fake, fake, fake, batch, 32, 8, 32 * 128, 2048, 2048 * 8 * 128, fake, 1 << 30, None)

    assert call_qk(wq=None) == -1 and b"gammas" in lib.anelm_last_error()    # the fused norm needs both gammas
    assert call_qk(tab_len=0) == -1 and b"table" in lib.anelm_last_error()
    assert call_qk(k_ld=1000) == -1                                            # k rows overlap
    assert call_qk(dt=7) == -1
    qa = lib.anelm_gqa_attention_qk_append

    def call_qa(wq=fake, k_ld=48 * 128, ws_bytes=1 << 30):
        row = 48 * 128
        return qa(fake, 1, fake, fake, fake, row, k_ld, row, wq, fake, 2, fake, fake, fake, 4096, 1e6, 1e-6, fake,
                  fake, fake, fake, 2, 32, 8, 32 * 128, 2048, 2048 * 8 * 128, fake, ws_bytes, None)

    # every check comes before the advance launch: a rejected call changes no ring
    assert call_qa(wq=None) == -1 and b"gqa_attention_qk_append" in lib.anelm_last_error()
    assert call_qa(k_ld=1000) == -1
    assert call_qa(ws_bytes=16) == -4 and b"workspace" in lib.anelm_last_error()
    adv = lib.anelm_kv_ring_advance
    assert adv(None, fake, 4, 2, 8, 2048, None) == -1
    assert adv(fake, fake, 4, 2, 3, 2048, None) == -1                          # groups' rings overlap
    assert adv(fake, fake, 4, 2, 8, 0, None) == -1
    assert adv(fake, fake, 0, 2, 8, 2048, None) == 0                           # nothing to do
    a = lib.anelm_kv_ring_append
    assert a(fake, fake, None, fake, fake, fake, 1024, 1024, 4, 8, 128, 2048, 2048 * 1024, None) == -1
    assert a(fake, fake, fake, fake, fake, fake, 1000, 1024, 4, 8, 128, 2048, 2048 * 1024, None) == -1  # k_ld < row


def test_projection_argument_checks(lib):
    """Validation of the projection entry points (no launch happens)."""
    P = ctypes.c_void_p
    fake, odd = P(0x1000), P(0x1008)
    f, x16, fu = lib.anelm_proj_f16, lib.anelm_proj_f16_x16, lib.anelm_proj_f16_fused
    assert f(fake, None, fake, 1, 64, 64, 64, 64, None) == -1
    assert f(fake, fake, fake, 0, 64, 64, 64, 64, None) == -1                   # batch 0
    assert f(fake, fake, fake, 2, 64, 64, 32, 64, None) == -1                   # ld_x < in_dim
    assert f(fake, fake, fake, 9, 64, 72, 72, 64, None) == -1                   # in_dim % 32 and batch > 8
    assert f(fake, odd, fake, 2, 64, 40, 40, 64, None) == -1                    # unaligned x, row path
    assert x16(fake, fake, fake, 4, 64, 48, 48, 64, None) == -1                 # in_dim not a multiple of 32
    assert x16(fake, fake, fake, 4, 64, 64, 68, 64, None) == -1                 # fp16 row stride not 16 bytes
    assert fu(fake, fake, fake, 17, 64, 64, 64, 60, None, 1e-6, 0, None) == -1  # ld_y < out_dim
    assert fu(fake, fake, fake, 1, 64, 64, 64, 64, None, 1e-6, 3, None) == -1   # no such epilogue
    assert fu(fake, fake, fake, 1, 64, 64, 64, 64, odd, 1e-6, 0, None) == -1    # unaligned gamma
    assert fu(fake, fake, fake, 1, 64, 64, 64, 64, None, 1e-6, 1, None) == -1   # residual add onto its own input
    assert b"residual" in lib.anelm_last_error()
    assert f(fake, P(0x10F0), fake, 1, 64, 64, 64, 64, None) == -1             # x starts inside y (64 floats at 0x1000)
    assert b"overlaps" in lib.anelm_last_error()
    assert x16(P(0x1040), fake, fake, 1, 64, 64, 64, 64, None) == -1           # y starts inside the fp16 x
    xf = lib.anelm_proj_f16_x16_fused
    assert xf(fake, fake, fake, 1, 64, 64, 64, 64, 4, None) == -1              # no such epilogue
    assert xf(fake, fake, fake, 1, 64, 48, 48, 64, 0, None) == -1              # in_dim not a multiple of 32
    assert xf(P(0x1040), fake, fake, 1, 64, 64, 64, 64, 3, None) == -1         # fp16 y inside x16
    assert xf(P(0x0F90), fake, fake, 1, 64, 64, 64, 64, 0, None) == -1         # fp32 y runs into x16
    assert lib.anelm_rmsnorm_f16(P(0x10C0), fake, fake, 2, 1, 64, 64, 64, 1e-6, None) == -1  # out16 inside x
    b = lib.anelm_gqa_attention_bounded
    assert b(fake, fake, fake, fake, fake, fake, 1, 32, 8, 128, 4096, 128, 4096, 2048, 2048 * 1024, 0, fake,
             1 << 30, None) == -1                                               # bound 0


def test_deltanet_argument_checks(lib):
    fake = ctypes.c_void_p(0x1000)
    assert lib.anelm_rmsnorm_gated(fake, fake, fake, fake, 5, 4, 1, 128, 128, 128, 128, 1e-6, None) == -1  # dtype
    assert lib.anelm_rmsnorm_gated(fake, fake, None, fake, 0, 4, 1, 128, 128, 128, 128, 1e-6, None) == -1
    assert lib.anelm_rmsnorm_gated(fake, fake, fake, fake, 0, 4, 16, 128, 1024, 2048, 2048, 1e-6, None) == -1  # ld
    assert lib.anelm_l2_normalize(fake, 4, 1, 128, 64, 1.0, None) == -1                                    # ld < dim
    assert lib.anelm_l2_normalize(fake, 4, 0, 128, 4096, 1.0, None) == -1                                  # heads
    assert lib.anelm_conv1d_update(fake, fake, fake, fake, fake, 2, 6144, 1, 6144, 6144, 6144 * 3, None) == -1
    assert lib.anelm_conv1d_update(fake, fake, None, fake, fake, 2, 6144, 4, 6144, 6144, 6144 * 3, None) == -1
    assert lib.anelm_conv1d_update(fake, fake, fake, fake, fake, 2, 6144, 4, 6144, 6144, 100, None) == -1  # overlap
    s = lib.anelm_ssm_step
    assert s(fake, fake, fake, fake, fake, fake, fake, 1, 16, 16, 96, 128, 2048, 2048, 2048, 16 * 128 * 128, None) == -1
    assert s(fake, fake, fake, fake, fake, fake, fake, 1, 16, 5, 128, 128, 2048, 2048, 2048, 16 * 128 * 128, None) == -1
    assert b"key_dim" in lib.anelm_last_error() or b"multiple" in lib.anelm_last_error()
    c = lib.anelm_conv_ssm_step_gated_norm
    n = 16 * 128
    ok = [fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, 0, 2, 16, 3 * n, n, n, 16 * 128 * 128, 3 * n * 3,
          ctypes.c_float(0.088), ctypes.c_float(1e-6), None]
    for i, v in ((3, None), (10, 7), (12, 0), (13, 3 * n - 128), (16, 16 * 128 * 128 - 4), (17, 3 * n * 3 - 1)):
        bad = list(ok)
        bad[i] = v                     # no ring positions / dtype / heads / overlapping x, state or ring rows
        assert c(*bad) == -1, i
    assert lib.anelm_matvec(None, fake, fake, 4, 4, None) == -1
    assert lib.anelm_matvec(fake, fake, fake, 4, 0, None) == -1


def test_rmsnorm_geometry_at_the_workload_shapes():
    """The row geometry (float4 per lane, lanes per row) that fixes the
    RMSNorm's summation order, at the decode and prefill shapes; a pure host
    query, so it runs here."""
    import anelm

    assert anelm.rmsnorm_geometry(1, 1024) == (1, 256)        # 0.6B decode: one float4 per lane
    assert anelm.rmsnorm_geometry(64, 2560) == (1, 640)       # 4B batched decode
    assert anelm.rmsnorm_geometry(2048, 1024) == (4, 64)      # 0.6B prefill: one wave per row
    assert anelm.rmsnorm_geometry(2048, 512) == (2, 64)       # also one wave, two float4 per lane
    assert anelm.rmsnorm_geometry(8192, 4096) == (2, 512)     # 8B prefill
    assert anelm.rmsnorm_geometry(4, 1022) == (0, 256)        # not a multiple of 4: the any-shape kernel
    with pytest.raises(anelm.AnelmError):
        anelm.rmsnorm_geometry(0, 1024)
