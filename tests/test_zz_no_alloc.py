"""sa_decode_noalloc (split partials in the library's own per-GPU scratch array) against sa_decode
with a caller workspace: same kernels, so the same bits, on two calls in a row (the second smaller,
so it reuses the scratch the first left behind), and as a step captured in a HIP graph and replayed;
plus the refusal of sizes past the scratch."""
import math
import sys

import pytest
import torch

from sparseattentioninfer_amd import _lib
from sparseattentioninfer_amd.patterns import decode_selection
from tests.helpers import seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _case(B, Hq, Hkv, D, page, lens, seed):
    nblk = [-(-L // page) for L in lens]
    P = sum(nblk) + 2
    kp = seeded((P, Hkv, page, D), seed, torch.bfloat16).to(DEV)
    vp = seeded((P, Hkv, page, D), seed + 1, torch.bfloat16).to(DEV)
    q = seeded((B, Hq, D), seed + 2, torch.bfloat16).to(DEV)
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(seed))
    table = torch.zeros(B, max(nblk), dtype=torch.int32)
    used = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[used:used + n].to(torch.int32)
        used += n
    sel, sel_off = decode_selection(B, Hkv, nblk, local=4, global_blocks=2, random_blocks=8, seed=seed)
    return q, kp, vp, table.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV), sel.to(DEV), sel_off.to(DEV)


def _args(q, kp, vp, table, lens, sel, sel_off, out, splits):
    B, Hq, D = q.shape
    Hkv, page = kp.shape[1], kp.shape[2]
    return [0, q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(),
            kp.stride(0), kp.stride(1), kp.stride(2),
            table.data_ptr(), table.stride(0), table.size(1), kp.size(0), lens.data_ptr(), 0,
            sel.data_ptr(), sel.stride(0), sel.stride(1), sel_off.data_ptr(), sel_off.stride(0), sel_off.stride(1),
            Hkv, out.data_ptr(), out.stride(0), out.stride(1), B, Hq, Hkv, D, page, 1.0 / math.sqrt(D), splits]


def test_noalloc_decode_equals_workspace_decode_twice():
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for call, (B, lens, splits) in enumerate([(8, [16384, 9000, 64, 1, 4097, 700, 12000, 300], 12),
                                              (3, [5000, 65, 2048], 5)]):
        _say(f"[noalloc] call {call}: B={B} splits={splits}")
        case = _case(B, 32, 8, 128, 64, lens, seed=50 + call)
        want = torch.empty_like(case[0])
        got = torch.full_like(case[0], float("nan"))
        need = int(lib.sa_decode_workspace_bytes(B, 32, 128, splits))
        assert 0 < need <= int(lib.sa_decode_noalloc_scratch_bytes())
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        st = lib.sa_decode(*_args(*case, want, splits), ws.data_ptr(), need, stream)
        assert st == 0, lib.sa_last_error()
        st = lib.sa_decode_noalloc(*_args(*case, got, splits), stream)
        assert st == 0, lib.sa_last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), f"call {call}: max diff {(got.float() - want.float()).abs().max()}"


def test_noalloc_decode_replays_in_a_graph():
    """The caller the entry point is for: a decode step captured in a HIP graph (split partials in the
    scratch array, then the combine kernel) gives the workspace decode's bits at every replay, with
    another sa_decode_noalloc call on other inputs run eagerly between the replays (it overwrites the
    scratch the replay then fills again)."""
    lib = _lib.load()
    B, lens, splits = 6, [9000, 64, 4097, 16384, 700, 3000], 7
    case = _case(B, 32, 8, 128, 64, lens, seed=61)
    other = _case(B, 32, 8, 128, 64, lens[::-1], seed=62)
    need = int(lib.sa_decode_workspace_bytes(B, 32, 128, splits))
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    want = torch.empty_like(case[0])
    want_other = torch.empty_like(other[0])
    cur = torch.cuda.current_stream().cuda_stream
    assert lib.sa_decode(*_args(*case, want, splits), ws.data_ptr(), need, cur) == 0, lib.sa_last_error()
    assert lib.sa_decode(*_args(*other, want_other, splits), ws.data_ptr(), need, cur) == 0, lib.sa_last_error()
    got = torch.full_like(case[0], float("nan"))
    got_other = torch.empty_like(other[0])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):   # warm-up outside the capture (the scratch address is looked up once)
        assert lib.sa_decode_noalloc(*_args(*case, got, splits), s.cuda_stream) == 0, lib.sa_last_error()
    torch.cuda.synchronize()
    _say("[noalloc] capture")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        assert lib.sa_decode_noalloc(*_args(*case, got, splits), s.cuda_stream) == 0, lib.sa_last_error()
    for rep in range(3):
        got.fill_(float("nan"))
        assert lib.sa_decode_noalloc(*_args(*other, got_other, splits), cur) == 0, lib.sa_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got_other, want_other), f"eager call before replay {rep}"
        _say(f"[noalloc] replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}: max diff {(got.float() - want.float()).abs().max()}"


def test_noalloc_refuses_sizes_past_its_scratch():
    lib = _lib.load()
    cap = int(lib.sa_decode_noalloc_scratch_bytes())
    B = cap // (16 * 32 * 130 * 4) + 1          # 16 splits of [B, 32, 130] fp32 partials exceed it
    assert lib.sa_decode_workspace_bytes(B, 32, 128, 16) > cap
    # NULL tensors: the size check returns first; were it ever to let the call through, sa_decode's
    # own NULL check would refuse it (a different status) before any launch
    null = None
    args = [0, null, 4096, 128, null, null, 8192, 8192, 128, null, 256, 256, 1 << 20, null, 0,
            null, 8 * 16, 16, null, 16, 2, 8, null, 4096, 128, B, 32, 8, 128, 64, 0.088, 16,
            torch.cuda.current_stream().cuda_stream]
    st = lib.sa_decode_noalloc(*args)
    assert st == -7 and b"scratch bytes" in lib.sa_last_error()
