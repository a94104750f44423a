"""The C ABI boundary on a CPU host: the library loads, exports every entry point
include/tilefoundry_amd.h declares, and every argument check fails with the
right status before any HIP call is made (no compute here)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tilefoundry_amd.h"
LIB = ROOT / "tilefoundry_amd" / "libtilefoundry_amd.so"

OK, NULL, SHAPE, ALIGN, CAPACITY, ARG, LAUNCH = range(7)


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(tfa_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail("libtilefoundry_amd.so is not built (python -m tilefoundry_amd._build)")
    L = ctypes.CDLL(str(LIB))
    L.tfa_last_error.restype = ctypes.c_char_p
    L.tfa_status_string.restype = ctypes.c_char_p
    L.tfa_lm_head_blocks.restype = ctypes.c_int64
    L.tfa_lm_head_blocks.argtypes = [ctypes.c_int64]
    return L


def test_every_declared_symbol_is_exported(lib):
    names = declared()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_status_strings(lib):
    assert lib.tfa_abi_version() == 1
    assert lib.tfa_status_string(OK) == b"ok"
    assert lib.tfa_status_string(SHAPE) == b"unsupported shape"
    assert lib.tfa_status_string(99) == b"unknown status"
    assert lib.tfa_lm_head_blocks(151936) == 9496


P = ctypes.c_void_p
I64 = ctypes.c_int64
F = ctypes.c_float
I = ctypes.c_int
BUF = ctypes.create_string_buffer(64)
A = ctypes.cast(ctypes.addressof(BUF) + (-ctypes.addressof(BUF)) % 16, P)   # 16-byte aligned host pointer
MIS = P(A.value + 2)                                                         # misaligned


def call(lib, name, *args):
    fn = getattr(lib, name)
    return fn(*args), lib.tfa_last_error().decode()


def test_norm_argument_checks(lib):
    st, msg = call(lib, "tfa_rms_norm", A, A, A, I64(4), I64(7), F(1e-6), I(0), P(None))
    assert st == SHAPE and "multiple of 8" in msg
    st, _ = call(lib, "tfa_rms_norm", A, A, A, I64(4), I64(16384), F(1e-6), I(0), P(None))
    assert st == SHAPE
    st, msg = call(lib, "tfa_rms_norm", A, A, A, I64(4), I64(2048), F(1e-6), I(3), P(None))
    assert st == ARG and "mode" in msg
    st, _ = call(lib, "tfa_rms_norm", P(None), A, A, I64(4), I64(2048), F(1e-6), I(0), P(None))
    assert st == NULL
    st, _ = call(lib, "tfa_rms_norm", MIS, A, A, I64(4), I64(2048), F(1e-6), I(0), P(None))
    assert st == ALIGN
    # zero rows: nothing to do, null pointers allowed, no launch
    st, _ = call(lib, "tfa_rms_norm", P(None), P(None), P(None), I64(0), I64(2048), F(1e-6), I(0), P(None))
    assert st == OK
    st, _ = call(lib, "tfa_add_rms_norm", A, P(None), A, A, A, I64(4), I64(2048), F(1e-6), I(0), P(None))
    assert st == NULL
    st, _ = call(lib, "tfa_resid_rms_norm_partials", A, A, I64(0), A, A, A, I64(2048), F(1e-6), P(None))
    assert st == SHAPE


def test_gemv_argument_checks(lib):
    st, msg = call(lib, "tfa_gemv", A, A, A, I64(64), I64(30), I(1), P(None))
    assert st == SHAPE and "multiple of 32" in msg
    st, _ = call(lib, "tfa_gemv", A, A, A, I64(0), I64(64), I(1), P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_gemv", A, MIS, A, I64(64), I64(64), I(1), P(None))
    assert st == ALIGN
    st, _ = call(lib, "tfa_gemv", A, A, P(None), I64(64), I64(64), I(1), P(None))
    assert st == NULL
    st, _ = call(lib, "tfa_gemv_residual", A, A, P(None), P(None), A, I64(64), I64(64), P(None))
    assert st == NULL
    st, _ = call(lib, "tfa_rmsnorm_gemv_swiglu", A, P(None), F(1e-6), A, A, I64(64), I64(64), P(None))
    assert st == NULL
    st, _ = call(lib, "tfa_lm_head_argmax", A, P(None), F(1e-6), A, I64(100), I64(64), P(None), A, A, P(None))
    assert st == NULL
    st, _ = call(lib, "tfa_sample_step", A, A, I64(0), A, A, A, A, A, I64(8), P(None), P(None))
    assert st == SHAPE
    st, msg = call(lib, "tfa_decode_qkv", A, P(None), P(None), I64(0), P(None), A, F(1e-6), A,
                   I64(2048), I64(3072), I64(1024), A, P(None), A, I64(64), P(None), P(None))
    assert st == NULL
    st, msg = call(lib, "tfa_decode_qkv", A, A, P(None), I64(1000), P(None), A, F(1e-6), A,
                   I64(2048), I64(3072), I64(1024), A, A, A, I64(64), P(None), P(None))
    assert st == NULL and "embed mode" in msg


def test_attention_argument_checks(lib):
    args = lambda hd, cap, split, hq=16, hkv=8: (A, P(None), I64(0), P(None), P(None), F(1e-6), P(None),
                                                  P(None), I64(0), A, A, P(None), A, I64(1), I64(hq),
                                                  I64(hkv), I64(hd), I64(cap), I64(split), F(0.088),
                                                  A, A, A, I(0), P(None), P(None))
    st, msg = call(lib, "tfa_decode_attention", *args(64, 512, 64))
    assert st == SHAPE and "128" in msg
    st, _ = call(lib, "tfa_decode_attention", *args(128, 500, 64))
    assert st == SHAPE
    st, _ = call(lib, "tfa_decode_attention", *args(128, 512, 64, hq=12, hkv=8))
    assert st == SHAPE
    st, msg = call(lib, "tfa_decode_attention", *args(128, 512, 16))
    assert st == SHAPE and "split" in msg
    fused = list(args(128, 512, 64))
    fused[3] = A  # gamma_q given, the rest of the fused-mode operands missing
    st, msg = call(lib, "tfa_decode_attention", *fused)
    assert st == NULL and "fused" in msg
    st, _ = call(lib, "tfa_attn_combine", A, A, A, A, I64(0), I64(1), I64(16), I64(128), P(None), I64(0), P(None))
    assert st == SHAPE
    part_only = list(args(128, 512, 64))
    part_only[0], part_only[1], part_only[2] = P(None), A, I64(1)   # partials without fused mode
    st, msg = call(lib, "tfa_decode_attention", *part_only)
    assert st == ARG and "partials" in msg


def test_mla_attention_argument_checks(lib):
    args = lambda heads, cap, split: (A, A, A, A, I64(8), I64(heads), I64(cap), I64(split), F(0.1), A, A, A,
                                      P(None), P(None))
    st, msg = call(lib, "tfa_mla_attention", *args(40, 8192, 48))   # not a multiple of 32
    assert st == SHAPE and "multiple of 128" in msg
    st, _ = call(lib, "tfa_mla_attention", *args(40, 8192, 160))   # past 128, not whole 128-position steps
    assert st == SHAPE
    st, _ = call(lib, "tfa_mla_attention", *args(40, 8192, 2048))
    assert st == SHAPE
    st, _ = call(lib, "tfa_mla_attention", *args(49, 8192, 256))
    assert st == SHAPE
    st, _ = call(lib, "tfa_mla_attention", *args(40, 8000, 256))
    assert st == SHAPE


def test_batched_argument_checks(lib):
    st, msg = call(lib, "tfa_skinny_gemm", A, A, I64(33), I64(64), I64(2048), I64(1), I(0), A, P(None), P(None), P(None), P(None), P(None))
    assert st == SHAPE and "[1, 32]" in msg
    st, _ = call(lib, "tfa_skinny_gemm", A, A, I64(32), I64(64), I64(2000), I64(1), I(0), A, P(None), P(None), P(None), P(None), P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_skinny_gemm", A, A, I64(32), I64(64), I64(2048), I64(2), I(1), P(None), A, P(None), P(None), P(None), P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_skinny_gemm", A, A, I64(32), I64(64), I64(2048), I64(1), I(7), A, A, A, A, A, P(None))
    assert st == ARG
    st, msg = call(lib, "tfa_skinny_gemm", A, A, I64(4), I64(64), I64(2048), I64(2), I(3), P(None), P(None), P(None), A, A, P(None))
    assert st == SHAPE and "ks=1" in msg
    st, _ = call(lib, "tfa_rms_norm_div", A, A, A, I64(4), I64(2560), F(1e-5), F(0.0), P(None))
    assert st == ARG
    st, _ = call(lib, "tfa_rms_norm_div", A, A, A, I64(4), I64(2561), F(1e-5), F(10.0), P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_rows_norm", P(None), P(None), I64(0), A, P(None), I64(1), A, A, A, I64(4), I64(2048), F(1e-6), P(None), P(None))
    assert st == NULL
    st, _ = call(lib, "tfa_batch_sample_step", A, A, I64(10), I64(0), A, A, A, A, A, I64(8), P(None), P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_copy_stream", A, A, I64(17), P(None))
    assert st == SHAPE


def test_prompt_prefill_argument_checks(lib):
    # f32 GEMM: n not a multiple of 128, k not of 64, a null operand
    st, msg = call(lib, "tfa_gemm_nt_f32", A, A, A, I64(37), I64(300), I64(2048), I64(2048), I64(2048), I64(300), P(None))
    assert st == SHAPE and "128" in msg
    st, _ = call(lib, "tfa_gemm_nt_f32", A, A, A, I64(37), I64(512), I64(100), I64(100), I64(100), I64(512), P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_gemm_nt_f32", P(None), A, A, I64(37), I64(512), I64(2048), I64(2048), I64(2048), I64(512), P(None))
    assert st == NULL
    # split f32 GEMM: splits that do not divide the k-tiles, too many splits
    st, msg = call(lib, "tfa_gemm_nt_f32_split", A, A, A, I64(37), I64(512), I64(2048), I64(2048), I64(2048),
                   I64(512), I64(3), P(None))
    assert st == SHAPE and "splits" in msg
    st, _ = call(lib, "tfa_gemm_nt_f32_split", A, A, A, I64(37), I64(512), I64(2048), I64(2048), I64(2048),
                 I64(512), I64(16), P(None))
    assert st == SHAPE
    # SwiGLU pairs: odd inter, ld too small, misaligned gu, bad split count; the
    # unsplit entry keeps its own argument list and checks the same shapes
    st, _ = call(lib, "tfa_swiglu_pairs_split", A, I64(1), I64(12288), I64(4), I64(6146), A, P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_swiglu_pairs_split", A, I64(1), I64(100), I64(4), I64(6144), A, P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_swiglu_pairs_split", MIS, I64(1), I64(12288), I64(4), I64(6144), A, P(None))
    assert st == ALIGN
    st, _ = call(lib, "tfa_swiglu_pairs_split", A, I64(9), I64(12288), I64(4), I64(6144), A, P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_swiglu_pairs", A, I64(12288), I64(4), I64(6146), A, P(None))
    assert st == SHAPE
    st, _ = call(lib, "tfa_swiglu_pairs", MIS, I64(12288), I64(4), I64(6144), A, P(None))
    assert st == ALIGN
    # q/k norm + RoPE rows: positions past the cache or the rope table, head_dim, split count
    qk = lambda n, pos0, cap, rope, hd=128, ks=1: (A, I64(ks), I64(4096), A, A, F(1e-6), A, A, I64(rope), I64(2),
                                                   I64(n), I64(pos0), A, A, I64(cap), A, I64(16), I64(8), I64(hd),
                                                   P(None))
    st, msg = call(lib, "tfa_prefill_qk_rope_split", *qk(100, 0, 512, 512, ks=0))
    assert st == SHAPE and "ks" in msg
    st, msg = call(lib, "tfa_prefill_qk_rope_split", *qk(100, 10, 100, 512))
    assert st == CAPACITY and "capacity" in msg
    st, msg = call(lib, "tfa_prefill_qk_rope_split", *qk(100, 0, 512, 64))
    assert st == CAPACITY and "rope" in msg
    st, _ = call(lib, "tfa_prefill_qk_rope_split", *qk(100, 0, 512, 512, hd=64))
    assert st == SHAPE
    st, _ = call(lib, "tfa_prefill_qk_rope_split", *qk(0, 0, 512, 512))
    assert st == SHAPE
    unsplit = lambda *a: (a[0],) + a[2:]   # the same arguments without ks
    st, msg = call(lib, "tfa_prefill_qk_rope", *unsplit(*qk(100, 10, 100, 512)))
    assert st == CAPACITY and "capacity" in msg
    st, _ = call(lib, "tfa_prefill_qk_rope", *unsplit(*qk(100, 0, 512, 512, hd=64)))
    assert st == SHAPE
    # causal attention: head_dim, empty n, heads not a multiple, misaligned stride
    ca = lambda n, hd=128, hq=16, hkv=8, q_rs=2048: (A, I64(q_rs), I64(128), I64(0), A, I64(1024), I64(128), I64(0),
                                                     A, I64(1024), I64(128), I64(0), A, I64(2048), I64(0), I64(1),
                                                     I64(n), I64(hq), I64(hkv), I64(hd), F(0.088), P(None))
    st, msg = call(lib, "tfa_causal_attention", *ca(64, hd=64))
    assert st == SHAPE and "128, 256" in msg
    st, _ = call(lib, "tfa_causal_attention", *ca(0))
    assert st == SHAPE
    st, _ = call(lib, "tfa_causal_attention", *ca(64, hq=12))
    assert st == SHAPE
    st, _ = call(lib, "tfa_causal_attention", *ca(64, q_rs=2044))
    assert st == ALIGN


def test_mla_prep_q_gemv_argument_checks(lib):
    # q_lora past 1024 or not a multiple of 32, an empty cache, a null cache, a misaligned partial
    args = lambda qa, cap=64, part=A, lat=A: (part, I64(qa), A, A, F(1e-6), A, A, I64(64), A, lat, A,
                                              I64(cap), A, A, I64(3840), P(None))
    st, msg = call(lib, "tfa_mla_prep_q_gemv", *args(1056))
    assert st == SHAPE and "1024" in msg
    st, _ = call(lib, "tfa_mla_prep_q_gemv", *args(100))
    assert st == SHAPE
    st, _ = call(lib, "tfa_mla_prep_q_gemv", *args(768, cap=0))
    assert st == SHAPE
    st, _ = call(lib, "tfa_mla_prep_q_gemv", *args(768, lat=P(None)))
    assert st == NULL
    st, _ = call(lib, "tfa_mla_prep_q_gemv", *args(768, part=MIS))
    assert st == ALIGN


def test_mla_qb_absorb_argument_checks(lib):
    # q_lora other than 768, a batch past 32, heads past 48, a null weight, a misaligned q_n
    args = lambda qa=768, b=8, h=40, wq=A, qn=A: (qn, I64(b), I64(h), I64(qa), wq, A, A, A, I64(64), A, A,
                                                  P(None), P(None))
    st, msg = call(lib, "tfa_mla_qb_absorb", *args(qa=512))
    assert st == SHAPE and "768" in msg
    st, _ = call(lib, "tfa_mla_qb_absorb", *args(b=33))
    assert st == SHAPE
    st, _ = call(lib, "tfa_mla_qb_absorb", *args(h=49))
    assert st == SHAPE
    st, _ = call(lib, "tfa_mla_qb_absorb", *args(wq=P(None)))
    assert st == NULL
    st, _ = call(lib, "tfa_mla_qb_absorb", *args(qn=MIS))
    assert st == ALIGN


def test_mla_prep_qb_absorb_argument_checks(lib):
    # q_lora other than 768, heads past 48, an empty cache, a null cache, a misaligned partial
    args = lambda qa=768, h=40, cap=64, part=A, lat=A: (part, I64(qa), A, A, F(1e-6), A, A, I64(64), A, lat, A,
                                                        I64(cap), A, A, I64(h), A, P(None), P(None))
    st, msg = call(lib, "tfa_mla_prep_qb_absorb", *args(qa=1024))
    assert st == SHAPE and "768" in msg
    st, _ = call(lib, "tfa_mla_prep_qb_absorb", *args(h=49))
    assert st == SHAPE
    st, _ = call(lib, "tfa_mla_prep_qb_absorb", *args(cap=0))
    assert st == SHAPE
    st, _ = call(lib, "tfa_mla_prep_qb_absorb", *args(lat=P(None)))
    assert st == NULL
    st, _ = call(lib, "tfa_mla_prep_qb_absorb", *args(part=MIS))
    assert st == ALIGN


def test_torch_extension_rejects_host_tensors():
    from tilefoundry_amd import ops

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    g = torch.ones(64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.rms_norm(x, g, 1e-6)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.gemv(torch.zeros(64, dtype=torch.bfloat16), torch.zeros(8, 64, dtype=torch.bfloat16))


def test_integration_stub_argtypes_match_the_header():
    """Every ctypes binding shown in INTEGRATION.md passes as many arguments as
    the header declares for that entry point."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {m.group(1): m.group(2) for m in re.finditer(r"\b(tfa_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S)}
    stub = (ROOT / "INTEGRATION.md").read_text()
    bound = re.findall(r"L\.(tfa_\w+)\.argtypes\s*=\s*\[([^\]]*)\]", stub, flags=re.S)
    assert len(bound) >= 8
    for name, args in bound:
        assert name in decls, f"{name} is bound in INTEGRATION.md but not declared"
        params = decls[name].strip()
        n_decl = 0 if params in ("", "void") else params.count(",") + 1
        n_stub = len([a for a in args.split(",") if a.strip()])
        assert n_stub == n_decl, f"{name}: {n_stub} argtypes, {n_decl} declared parameters"
