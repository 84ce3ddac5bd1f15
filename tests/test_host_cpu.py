"""Host-side checks that need no GPU: the C library loads and exports every
function of include/fa2_mi355x.h, the ctypes mirror matches the C struct
layout, argument validation rejects bad calls before touching the device, and
the Python drop-in module keeps the reference's API, eligibility predicate
and fallback behaviour (reference @ None: flash_attn_v100_cuda.py:59-166,
train.py:87-113, 1946-1961)."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fa2_capi as capi

REPO = capi.REPO


def test_library_exports_every_header_function():
    lib = capi.load()
    names = capi.header_functions()
    assert set(names) >= {"fa2_fwd_f16", "fa2_bwd_f16", "fa2_bwd_workspace_bytes", "fa2_rope_f16",
                          "fa2_status_string", "fa2_last_error", "fa2_version"}
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert b"gfx950" in lib.fa2_version()


def test_struct_layout_matches_header(tmp_path):
    """Compile the header with gcc and compare sizeof/offsetof with ctypes."""
    src = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{capi.HEADER}"', "int main(void){"]
    for cname, cls in capi.STRUCTS.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(src)], check=True)
    out = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], check=True, capture_output=True,
                                                        text=True).stdout.split("\n") if l)
    for cname, cls in capi.STRUCTS.items():
        assert int(out[cname]) == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert int(out[f"{cname}.{fname}"]) == getattr(cls, fname).offset, f"{cname}.{fname}"


def _dummy_fwd(**kw):
    p = capi.FwdParams()
    base = 1 << 20  # never dereferenced: every case fails validation first
    p.q = p.k = p.v = p.o = p.lse = base
    for f in ("q_stride", "k_stride", "v_stride", "o_stride"):
        setattr(p, f, capi.I64x3(64 * 8 * 16, 64 * 16, 64))
    p.lse_stride = capi.I64x2(8 * 16, 16)
    p.B, p.H, p.S, p.D = 2, 8, 16, 64
    p.softmax_scale, p.dropout_p, p.seed, p.causal = 0.125, 0.0, 0, 1
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("field,value,status", [
    ("D", 128, 2), ("S", -1, 2), ("q", 0, 1), ("lse", 0, 1), ("k", (1 << 20) + 8, 3),
    ("v_stride", capi.I64x3(64 * 8 * 16, 64 * 16, 68), 3), ("q_stride", capi.I64x3(0, 0, 1 << 24), 2),
    ("dropout_p", 1.0, 4),
    ("dropout_p", -0.1, 4), ("softmax_scale", float("nan"), 4),
])
def test_fwd_validation_rejects_before_launch(field, value, status):
    lib = capi.load()
    p = _dummy_fwd(**{field: value})
    rc = lib.fa2_fwd_f16(ctypes.byref(p), None)
    assert rc == status, (rc, lib.fa2_last_error())
    assert lib.fa2_last_error() != b""
    assert lib.fa2_status_string(rc) != b"unknown status"


@pytest.mark.parametrize("s_k,coff,status", [(0, 0, 2), (-5, 0, 2), (16, (1 << 30) + 1, 4), (16, -(1 << 30) - 1, 4)])
def test_fwd_kv_validation_rejects_before_launch(s_k, coff, status):
    lib = capi.load()
    p = _dummy_fwd()
    rc = lib.fa2_fwd_kv_f16(ctypes.byref(p), s_k, coff, None)
    assert rc == status, (rc, lib.fa2_last_error())
    # B*H*s_k must fit the kernels' int32 row indices
    p = _dummy_fwd()
    assert lib.fa2_fwd_kv_f16(ctypes.byref(p), 1 << 28, 0, None) == 2


def test_fwd_kv_split_validation():
    lib = capi.load()
    assert lib.fa2_fwd_kv_workspace_bytes(2, 3, 5, 4) == 4 * 2 * 3 * 5 * 66 * 4
    assert lib.fa2_fwd_kv_workspace_bytes(2, 3, 5, 1) == 0
    p = _dummy_fwd()
    for nsplit, status in ((0, 4), (1025, 4), (4, 5)):   # bad counts; nsplit > 1 without a workspace
        rc = lib.fa2_fwd_kv_split_f16(ctypes.byref(p), 64, 0, nsplit, None, 0, None)
        assert rc == status, (nsplit, rc, lib.fa2_last_error())
    # B*H*S within limits, but B*H*ceil(S/128)*nsplit past the int32 grid: rejected as a shape
    p = _dummy_fwd(B=1 << 22, H=1, S=2)
    rc = lib.fa2_fwd_kv_split_f16(ctypes.byref(p), 64, 0, 1024, None, 0, None)
    assert rc == 2, (rc, lib.fa2_last_error())


def test_empty_problem_is_a_noop():
    lib = capi.load()
    for dim in ("B", "H", "S"):
        p = _dummy_fwd(**{dim: 0})
        assert lib.fa2_fwd_f16(ctypes.byref(p), None) == 0
    # fp32 delta and LSE (rounded to 256 B), fp32 row terms (8 B per query, S rounded to 32,
    # rounded to 256 B), fp32 dQ accumulator
    assert lib.fa2_bwd_workspace_bytes(2, 3, 5) == 256 + 2 * 3 * 32 * 8
    assert lib.fa2_bwd_workspace_bytes(1, 1, 33) == 512 + 512
    assert lib.fa2_bwd_workspace_bytes(0, 3, 5) == 0


def test_dropout_mask_size_and_validation():
    """Keep-bit words: per (b, h), 2*ceil(S/128) 64-key tiles x 2 halves x S rounded up to 256
    rows, 4 bytes each; a misaligned mask is rejected only when dropout would use it, and the
    fa2_fwd_kv_* entry points take none."""
    lib = capi.load()
    assert lib.fa2_dropout_mask_bytes(1, 1, 1) == 2 * 2 * 256 * 4
    assert lib.fa2_dropout_mask_bytes(8, 12, 4096) == 96 * 64 * 2 * 4096 * 4
    assert lib.fa2_dropout_mask_bytes(2, 3, 257) == 6 * 6 * 2 * 512 * 4
    assert lib.fa2_dropout_mask_bytes(0, 3, 5) == 0 and lib.fa2_dropout_mask_bytes(1, 1, -1) == 0
    # causal: 128-key block j keeps 4 runs (2 tiles x 2 halves) of R - 128 j words
    assert lib.fa2_dropout_mask_bytes_causal(1, 1, 1) == 4 * 256 * 4
    assert lib.fa2_dropout_mask_bytes_causal(2, 3, 257) == 6 * 4 * (512 + 384 + 256) * 4
    assert lib.fa2_dropout_mask_bytes_causal(8, 12, 4096) == 96 * 4 * sum(4096 - 128 * j for j in range(32)) * 4
    assert lib.fa2_dropout_mask_bytes_causal(0, 3, 5) == 0
    p = _dummy_fwd(dropout_p=0.1, dropout_mask=(1 << 21) + 4)
    assert lib.fa2_fwd_f16(ctypes.byref(p), None) == 3, lib.fa2_last_error()
    assert b"dropout_mask" in lib.fa2_last_error()
    p = _dummy_fwd(dropout_mask=1 << 21)
    assert lib.fa2_fwd_kv_f16(ctypes.byref(p), 16, 0, None) == 4
    assert lib.fa2_fwd_kv_split_f16(ctypes.byref(p), 16, 0, 2, None, 0, None) == 4
    pb = capi.BwdParams()
    base = 1 << 20
    pb.q = pb.k = pb.v = pb.o = pb.dout = pb.lse = pb.dq = pb.dk = pb.dv = base
    for f in ("q_stride", "k_stride", "v_stride", "o_stride", "do_stride", "dq_stride", "dk_stride", "dv_stride"):
        setattr(pb, f, capi.I64x3(64 * 64, 64 * 64, 64))
    pb.lse_stride = capi.I64x2(64, 64)
    pb.B, pb.H, pb.S, pb.D, pb.softmax_scale, pb.dropout_p = 1, 1, 64, 64, 0.125, 0.1
    pb.dropout_mask = base + 8
    need = lib.fa2_bwd_workspace_bytes(1, 1, 64)
    assert lib.fa2_bwd_f16(ctypes.byref(pb), 7, ctypes.c_void_p(1 << 22), need, None) == 3
    assert b"dropout_mask" in lib.fa2_last_error()
    # An undersized mask buffer (the device writes would run past it) is rejected before any
    # launch, in the forward and the backward; its size only matters when dropout uses it.
    fwd_need = lib.fa2_dropout_mask_bytes_causal(2, 8, 16)   # _dummy_fwd is causal
    p = _dummy_fwd(dropout_p=0.1, dropout_mask=1 << 21, dropout_mask_bytes=fwd_need - 4)
    assert lib.fa2_fwd_f16(ctypes.byref(p), None) == 5, lib.fa2_last_error()
    assert b"dropout_mask needs" in lib.fa2_last_error()
    pb.dropout_mask, pb.dropout_mask_bytes = base, lib.fa2_dropout_mask_bytes(1, 1, 64) - 16
    assert lib.fa2_bwd_f16(ctypes.byref(pb), 7, ctypes.c_void_p(1 << 22), need, None) == 5
    assert b"dropout_mask needs" in lib.fa2_last_error()
    pb.dropout_p = 0.0     # no dropout: the mask is not used, so its size is not checked
    assert lib.fa2_bwd_f16(ctypes.byref(pb), 0, ctypes.c_void_p(1 << 22), need, None) == 0


# p values: the tests' own, values whose p * 2^24 is not an integer, values next to a
# multiple of 2^-24, and the extremes of [0, 1).
THRESHOLD_PS = [0.1, 0.25, 0.5, 0.9, 1 / 3, 0.123456789, 0.7, 5e-8, 2.0 ** -24, 3 * 2.0 ** -24,
                float(np.nextafter(np.float32(0.5), np.float32(1))),
                float(np.nextafter(np.float32(0.5), np.float32(0))), 0.0, 0.99999994]


@pytest.mark.parametrize("p", THRESHOLD_PS)
def test_dropout_threshold_equals_reference_fp32_compare_exhaustively(p):
    """Every kernel keeps an element iff (h >> 8) >= fa2_dropout_threshold(p); the reference
    keeps it iff (h >> 8) * 2^-24 >= p in fp32 (fa_common.cuh:37).  Both over all 2^24
    values of h >> 8."""
    lib = capi.load()
    thr = lib.fa2_dropout_threshold(p)
    v = np.arange(1 << 24, dtype=np.uint32)
    ref = v.astype(np.float32) * np.float32(1.0 / 16777216.0) >= np.float32(p)
    assert np.array_equal(ref, v >= thr), (p, thr)


def test_bwd_noalloc_rejects_before_any_hip_call():
    """The allocation-free backward checks its size limit and mode before touching the
    device (it would otherwise look up its scratch array on the current GPU)."""
    lib = capi.load()
    assert lib.fa2_bwd_noalloc_scratch_bytes(2, 3, 5) == 256 + 2 * 3 * 32 * 8
    assert lib.fa2_bwd_noalloc_scratch_bytes(0, 3, 5) == 0
    p = capi.BwdParams()
    p.B, p.H, p.S, p.D, p.softmax_scale = 64, 64, 4096, 64, 0.125
    assert lib.fa2_bwd_f16_noalloc(ctypes.byref(p), 7, None) == 5
    assert b"FA2_BWD_SCRATCH_MAX_BYTES" in lib.fa2_last_error()
    p.S = 64
    assert lib.fa2_bwd_f16_noalloc(ctypes.byref(p), 8, None) == 4    # modes are 0..7
    assert lib.fa2_bwd_f16_noalloc(ctypes.byref(p), 16, None) == 4   # bad mode
    assert lib.fa2_bwd_f16_noalloc(ctypes.byref(p), 0, None) == 0    # nothing requested
    assert lib.fa2_bwd_f16_noalloc(None, 7, None) == 1


def test_bwd_validation():
    lib = capi.load()
    p = capi.BwdParams()
    p.B, p.H, p.S, p.D, p.softmax_scale = 1, 1, 64, 64, 0.125
    assert lib.fa2_bwd_f16(ctypes.byref(p), 16, None, 0, None) == 4         # bad mode
    assert lib.fa2_bwd_f16(ctypes.byref(p), 7, None, 0, None) == 5          # no workspace
    assert lib.fa2_bwd_f16(ctypes.byref(p), 7, ctypes.c_void_p(1 << 20), 16, None) == 5  # too small
    assert lib.fa2_bwd_f16(ctypes.byref(p), 0, None, 0, None) == 0          # nothing requested
    assert lib.fa2_bwd_f16(None, 7, None, 0, None) == 1


# ---------------------------------------------------------------------------
# Python drop-in module
# ---------------------------------------------------------------------------
import flash_attn_v100_cuda as fa  # noqa: E402


def test_module_api_surface():
    for name in ("is_available", "build_error", "can_use", "flash_attn_v100", "rope_can_use", "rope",
                 "_next_seed", "_fa_ready", "sdpa"):
        assert callable(getattr(fa, name)), name


def test_extension_loads_on_host():
    assert fa.is_available(), fa.build_error()
    ext = fa.extension()
    for op in ("fa_fwd", "fa_bwd", "rope_fwd", "rope_bwd"):
        assert hasattr(ext, op)


def test_cpu_tensors_are_ineligible_and_rejected():
    q = torch.randn(1, 2, 64, 64, dtype=torch.float16)
    assert not fa.can_use(q, q, q)
    with pytest.raises(ValueError):
        fa.flash_attn_v100(q, q, q)
    cos = torch.zeros(64, 64)
    assert not fa.rope_can_use(q, q, cos, cos)


def test_sdpa_shim_falls_back_bitwise_on_cpu():
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 4, 256, 64, generator=g) for _ in range(3))
    for kw in (dict(is_causal=True), dict(is_causal=False), dict(attn_mask=torch.ones(256, 256, dtype=torch.bool))):
        ref = F.scaled_dot_product_attention(q, k, v, **kw)
        assert torch.equal(fa.sdpa(q, k, v, **kw), ref)


def test_disable_switch_forces_sdpa(monkeypatch):
    monkeypatch.setenv("FA_V100_DISABLE", "1")
    q = torch.randn(1, 1, 8, 64)
    assert torch.equal(fa.sdpa(q, q, q, is_causal=True),
                       F.scaled_dot_product_attention(q, q, q, is_causal=True))


def test_missing_build_reports_and_raises(monkeypatch):
    """A missing extension must surface as is_available()==False plus a
    build_error() text (train.py:88-95 prints it and falls back), and the op
    itself must raise instead of silently computing on the CPU."""
    monkeypatch.setattr(fa, "_EXT", None)
    monkeypatch.setattr(fa, "_BUILD_ERROR", ImportError("not built"))
    assert not fa.is_available()
    assert "not built" in str(fa.build_error())
    with pytest.raises(RuntimeError):
        fa.extension()
    with pytest.raises(RuntimeError):
        fa._FlashAttnV100Cuda.forward(None, None, None, None, 0.0, True, 0.125)


def test_build_failure_path_in_fresh_process(tmp_path):
    """Point the loader at an empty lib dir in a fresh interpreter."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import flash_attn_v100_cuda as fa\n"
        "fa._LIB_DIR = %r\n"
        "print(fa.is_available(), type(fa.build_error()).__name__)\n"
    ) % (os.path.join(REPO, "universal-lm-trainer_amd"), str(tmp_path))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True).stdout
    assert out.split() == ["False", "ImportError"]


def test_eligibility_predicate_matches_reference_rules():
    """_fa_ready: fp16, 4-D, D=64, unit last stride, 32-byte base and strides."""
    class Fake:
        def __init__(self, dtype=torch.float16, shape=(1, 2, 8, 64), stride=(1024, 512, 64, 1), ptr=0):
            self.is_cuda, self.dtype, self._shape, self._stride, self._ptr = True, dtype, shape, stride, ptr

        def dim(self):
            return len(self._shape)

        def size(self, i):
            return self._shape[i]

        def stride(self, i=None):
            return self._stride if i is None else self._stride[i]

        def data_ptr(self):
            return self._ptr

        @property
        def shape(self):
            return torch.Size(self._shape)

    assert fa._fa_ready(Fake())
    assert not fa._fa_ready(Fake(dtype=torch.float32))
    assert not fa._fa_ready(Fake(shape=(1, 2, 8, 128), stride=(2048, 1024, 128, 1)))
    assert not fa._fa_ready(Fake(stride=(1024, 512, 64, 2)))
    assert not fa._fa_ready(Fake(ptr=16))
    assert not fa._fa_ready(Fake(stride=(1024, 520, 64, 1)))   # 1040 B not 32B-aligned
    # train.py layouts: q/k dense [B,S,H,D] view (row stride 768), v view of fused qkv (2304)
    assert fa._fa_ready(Fake(shape=(2, 12, 16, 64), stride=(16 * 768, 64, 768, 1)))
    assert fa._fa_ready(Fake(shape=(2, 12, 16, 64), stride=(16 * 2304, 64, 2304, 1), ptr=2 * 768 * 2))


def test_seed_counter_against_reference_vectors(monkeypatch):
    """The drop-in module's _next_seed, from a fresh counter, returns the seeds
    the reference's own _next_seed returned for the same initial seed
    (tests/golden/seed_golden.json, written by make_seed_golden.py)."""
    import itertools
    import json
    with open(os.path.join(os.path.dirname(__file__), "golden", "seed_golden.json")) as f:
        cases = json.load(f)["cases"]
    for c in cases:
        monkeypatch.setattr(torch.cuda, "initial_seed", lambda v=c["initial_seed"]: v)
        monkeypatch.setattr(fa, "_SEED_COUNTER", itertools.count(1))
        assert [fa._next_seed() for _ in c["seeds"]] == c["seeds"]


def test_decoder_kv_cache_matches_full_forward_on_cpu():
    """The decoder's KV-cache inference path (prefill, decode steps, a chunk) on the SDPA fallback
    equals a full-sequence forward at every position, in fp32 on the CPU."""
    import fa2_decoder as dec
    torch.manual_seed(0)
    m = dec.Decoder(vocab=100, d_model=128, n_heads=2, n_layers=2, d_ff=64, fa=None, use_kernel=False).eval()
    ids = dec.synthetic_ids(2, 40, vocab=100, seed=2)[:, :40]
    with torch.no_grad():
        full = m.forward(ids)
        cache = m.new_cache()
        outs = [m.forward_cached(ids[:, a:b], cache, 40) for a, b in ((0, 17), (17, 18), (18, 19), (19, 33), (33, 40))]
    got = torch.cat(outs, dim=1)
    assert torch.allclose(got, full, rtol=1e-4, atol=1e-5), (got - full).abs().max()


def test_python_mask_size_matches_c_abi(monkeypatch):
    """The autograd wrapper sizes the keep-bit words with the C ABI's formula, and a malformed
    FA_V100_DROPOUT_MASK_MAX_BYTES falls back to the default cap instead of failing the import."""
    lib = capi.load()
    for B, H, S in ((1, 1, 1), (2, 3, 257), (8, 12, 4096), (1, 2, 16384), (3, 5, 1000)):
        assert fa.dropout_mask_bytes(B, H, S) == lib.fa2_dropout_mask_bytes(B, H, S), (B, H, S)
        assert fa.dropout_mask_bytes(B, H, S, causal=True) == lib.fa2_dropout_mask_bytes_causal(B, H, S), (B, H, S)
    monkeypatch.setenv("FA_V100_DROPOUT_MASK_MAX_BYTES", "lots")
    assert fa._mask_cap() == 1 << 30
    monkeypatch.setenv("FA_V100_DROPOUT_MASK_MAX_BYTES", "0")
    assert fa._mask_cap() == 0


def test_bench_step_roofline():
    """bench.py's whole-step roofline: config 2 (B=8 H=12 S=4096) is MFMA-bound at 1188.5
    flop/B on the operation's minimum bytes (12 fp16 tensors + 2 fp32 rows); the S=512 bucket
    of config 3 (B=64) is HBM-bound there at 8 TB/s x 148.6 flop/B = 1188.5 TFLOP/s."""
    import bench
    f2 = 7 * 8 * 12 * 4096 * 4096 * 64
    r = bench.step_roofline(8, 12, 4096, f2, 700.0)
    assert r["minimum"]["algorithmic_bytes"] == 12 * 8 * 12 * 4096 * 128 + 2 * 8 * 12 * 4096 * 4
    assert r["minimum"]["bound"] == "mfma" and r["minimum"]["attainable"] == round(bench.PEAK_TFLOPS, 1)
    assert abs(r["minimum"]["intensity_flop_per_byte"] - 1188.5) < 0.1
    r = bench.step_roofline(64, 12, 512, 7 * 64 * 12 * 512 * 512 * 64, 360.0)
    assert r["minimum"]["bound"] == "hbm" and abs(r["minimum"]["attainable"] - 1188.5) < 0.1
    assert r["split_design"]["algorithmic_bytes"] == 16 * 64 * 12 * 512 * 128 + 8 * 64 * 12 * 512 * 4
    assert abs(r["minimum"]["frac"] - 360.0 / r["minimum"]["attainable"]) < 1e-4


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 exits with a nonzero status and says why."""
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU only" in r.stdout + r.stderr
