"""The no-allocation entry point, through the C ABI: tfa_rope_attend_noalloc
(split partials in the library's static device array) against tfa_rope_attend
(the same kernels over a caller's workspace) on the same inputs, bit for bit,
on two calls in a row -- the second smaller, so stale partials of the first
call would show -- plus the capacity limit, refused before any launch."""
import ctypes
from pathlib import Path

import pytest
import torch

from tests._check import assert_equal

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "tilefoundry_amd" / "libtilefoundry_amd.so"
BF = torch.bfloat16
P, I64 = ctypes.c_void_p, ctypes.c_int64
CAPACITY = 4


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(str(LIB))
    L.tfa_last_error.restype = ctypes.c_char_p
    L.tfa_rope_attend_splits.restype = ctypes.c_int64
    L.tfa_rope_attend_splits.argtypes = [ctypes.c_int64]
    L.tfa_rope_attend_noalloc_max_floats.restype = ctypes.c_int64
    return L


def _case(dev, heads, cap, ctx, pos, seed, nope=64, rope=32, v_dim=64):
    g = torch.Generator().manual_seed(seed)
    qk = nope + rope

    def r(*shape):
        return torch.randn(*shape, generator=g).to(BF).to(dev)

    inv = 1.0 / (10000.0 ** (torch.arange(0, rope, 2).float() / rope))
    ph = torch.outer(torch.arange(pos + 1).float(), inv)
    ph = torch.cat((ph, ph), -1)
    return {
        "q_up": r(heads, qk), "kv_up": r(heads, nope + v_dim), "k_rope": r(rope),
        "cos": ph.cos().to(BF).to(dev), "sin": ph.sin().to(BF).to(dev),
        "pos": torch.tensor([pos], dtype=torch.int32, device=dev),
        "k_cache": r(cap, heads, qk), "v_cache": r(cap, heads, v_dim),
        "ctx": torch.tensor([ctx], dtype=torch.int32, device=dev),
        "scale": torch.tensor([qk ** -0.5]).to(BF).to(dev),
        "heads": heads, "nope": nope, "rope": rope, "v_dim": v_dim, "cap": cap,
    }


def _out(c, dev):
    h = c["heads"]
    return (torch.full((h * c["v_dim"],), float("nan"), device=dev).to(BF),
            torch.zeros(h * (c["nope"] + c["rope"]), dtype=BF, device=dev),
            torch.zeros(h * c["v_dim"], dtype=BF, device=dev), torch.zeros(1, dtype=torch.int32, device=dev))


def _lead(c):
    return [P(c["q_up"].data_ptr()), P(c["kv_up"].data_ptr()), P(c["k_rope"].data_ptr()),
            P(c["cos"].data_ptr()), P(c["sin"].data_ptr()), I64(c["cos"].shape[0]), P(c["pos"].data_ptr()),
            P(c["k_cache"].data_ptr()), P(c["v_cache"].data_ptr()), I64(c["cap"]), P(c["ctx"].data_ptr()),
            P(c["scale"].data_ptr()), I64(c["heads"]), I64(c["nope"]), I64(c["rope"]), I64(c["v_dim"])]


def _with_workspace(lib, c, dev):
    ns = lib.tfa_rope_attend_splits(c["cap"])
    h = c["heads"]
    op = torch.empty(max(ns, 1) * h * c["v_dim"], device=dev)
    mp = torch.empty(max(ns, 1) * h, device=dev)
    lp = torch.empty(max(ns, 1) * h, device=dev)
    attn, k_new, v_new, err = _out(c, dev)
    stream = P(torch.cuda.current_stream(dev).cuda_stream)
    st = lib.tfa_rope_attend(*_lead(c), P(op.data_ptr()), P(mp.data_ptr()), P(lp.data_ptr()),
                             P(attn.data_ptr()), P(k_new.data_ptr()), P(v_new.data_ptr()), P(err.data_ptr()),
                             stream)
    assert st == 0, lib.tfa_last_error()
    return attn, k_new, v_new, err


def _no_alloc(lib, c, dev):
    attn, k_new, v_new, err = _out(c, dev)
    stream = P(torch.cuda.current_stream(dev).cuda_stream)
    st = lib.tfa_rope_attend_noalloc(*_lead(c), P(attn.data_ptr()), P(k_new.data_ptr()), P(v_new.data_ptr()),
                                     P(err.data_ptr()), stream)
    assert st == 0, lib.tfa_last_error()
    return attn, k_new, v_new, err


@pytest.mark.gpu
def test_no_alloc_equals_workspace_entry_twice(lib, dev):
    """Call 1: MiniCPM3's 40 heads over 3000 of 4096 cached rows (12 splits);
    call 2: 8 heads over 300 of 512 rows (2 splits) -- smaller, so anything the
    second call read from the first call's partials would differ."""
    cases = [_case(dev, heads=40, cap=4096, ctx=3000, pos=3000, seed=1),
             _case(dev, heads=8, cap=512, ctx=300, pos=300, seed=2)]
    for i, c in enumerate(cases):
        print(f"[case] no-alloc call {i + 1}: heads {c['heads']}, cap {c['cap']}, ctx {int(c['ctx'][0])}",
              flush=True)
        want = _with_workspace(lib, c, dev)
        got = _no_alloc(lib, c, dev)
        torch.cuda.synchronize()
        for name, a, b in zip(("attn", "k_new", "v_new", "err"), got, want):
            assert_equal(f"call {i + 1} {name}", a, b)
        assert not bool(torch.isnan(got[0].float()).any())
        assert int(got[3].item()) == 0


@pytest.mark.gpu
def test_no_alloc_empty_context_needs_no_scratch(lib, dev):
    """A zero-row cache launches only the merge (the token attends itself)."""
    c = _case(dev, heads=4, cap=0, ctx=0, pos=5, seed=3)
    c["k_cache"] = c["v_cache"] = torch.empty(0, dtype=BF, device=dev)
    want = _with_workspace(lib, c, dev)
    got = _no_alloc(lib, c, dev)
    torch.cuda.synchronize()
    for name, a, b in zip(("attn", "k_new", "v_new"), got, want):
        assert_equal(f"empty context {name}", a, b)


def test_no_alloc_refuses_beyond_the_array(lib):
    """Sizes past the array are refused with TFA_ERR_CAPACITY before any HIP call
    (host pointers are never dereferenced)."""
    maxf = lib.tfa_rope_attend_noalloc_max_floats()
    assert maxf == 1 << 20
    heads, v_dim = 40, 64
    ns_ok = maxf // (heads * (v_dim + 2))
    cap_bad = (ns_ok + 1) * 256
    buf = ctypes.create_string_buffer(64)
    a = P(ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16)
    args = [a, a, a, a, a, I64(1), a, a, a, I64(cap_bad), a, a, I64(heads), I64(64), I64(32), I64(v_dim),
            a, a, a, a, P(None)]
    st = lib.tfa_rope_attend_noalloc(*args)
    assert st == CAPACITY and b"scratch" in lib.tfa_last_error()
