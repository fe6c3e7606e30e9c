"""The C-ABI library loads on the CPU and exports every entry point the header declares."""
import ctypes
import re
from pathlib import Path

import pytest

from sparseattentioninfer_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"\b(sa_[a-z0-9_]+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        from sparseattentioninfer_amd import _build
        _build.build(verbose=False)
    return _lib.load()


def test_header_declares_entry_points():
    assert {"sa_abi_version", "sa_last_error", "sa_prefill", "sa_prefill_workspace_bytes", "sa_decode",
            "sa_decode_workspace_bytes", "sa_csr_to_tiles", "sa_block_mask_to_csr"} <= _declared()


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(str(_lib.library_path()))
    for name in sorted(_declared()):
        assert hasattr(raw, name), f"{name} declared in include/ but not exported"
    assert set(_lib.SIGNATURES) == _declared()


def test_abi_version_and_error_string(lib):
    assert lib.sa_abi_version() == _lib.ABI_VERSION
    assert isinstance(lib.sa_last_error(), bytes)


def test_argument_errors_are_reported_without_a_gpu(lib):
    # rejected before any HIP call: unsupported head dim
    st = lib.sa_prefill(0, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0,
                        None, 0, None, 0, None, 0, 4, 1, 1, 4, 4, 64, 64, 96, 64, 0, 0.1, None, 0, None)
    assert st == -3 and b"head dim 96" in lib.sa_last_error()
    # block sizes 16 / 32 need a tile schedule (tile masks), 64 / 128 take none
    st = lib.sa_prefill(0, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0,
                        None, 0, None, 0, None, 0, 4, 1, 1, 4, 4, 64, 64, 128, 16, 0, 0.1, None, 0, None)
    assert st == -4 and b"needs tile masks" in lib.sa_last_error()
    st = lib.sa_prefill(0, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0,
                        None, 0, None, 0, 8, 1, 4, 1, 1, 4, 4, 64, 64, 128, 64, 0, 0.1, None, 0, None)
    assert st == -4 and b"takes no tile masks" in lib.sa_last_error()
    st = lib.sa_csr_to_tiles(None, 0, None, 0, 2, 4, 64, None, None, 0, 4, None, 0, None, None)
    assert st == -4 and b"not 16 or 32" in lib.sa_last_error()
    st = lib.sa_csr_to_tiles(None, 0, None, 0, 2, 4, 16, None, None, 0, 4, None, 0, None, None)
    assert st == -6
    # GPU CSR builder: the write pass needs a width and a status word; NULL mask refused
    st = lib.sa_block_mask_to_csr(None, 0, 0, 2, 4, 4, None, 0, None, 8, 4, 0, None, None)
    assert st == -2 and b"width >= 1" in lib.sa_last_error()
    st = lib.sa_block_mask_to_csr(None, 0, 0, 2, 4, 4, None, 0, None, None, 0, 0, None, None)
    assert st == -6
    # one wave per (row, query block) in one launch: past 2^32 grid threads it is refused, not truncated
    st = lib.sa_block_mask_to_csr(None, 0, 0, 1 << 15, 1 << 12, 1, None, 0, None, None, 0, 0, None, None)
    assert st == -2 and b"one launch covers" in lib.sa_last_error()
    st = lib.sa_decode(0, None, 0, 0, None, None, 0, 0, 0, None, 0, 0, 0, None, 0, None, 0, 0, None, 0, 0,
                       3, None, 0, 0, 1, 4, 2, 128, 64, 0.1, 1, None, 0, None)
    assert st == -5 and b"sel_rows=3" in lib.sa_last_error()
    # a paged table narrower than its own column count is refused before anything is read
    fake = 16   # 16-byte aligned stand-in addresses; the call returns before any device access
    st = lib.sa_decode(0, fake, 8, 8, fake, fake, 8, 8, 8, fake, 4, 8, 10, fake, 0, fake, 0, 0, fake, 0, 0,
                       2, fake, 8, 8, 1, 4, 2, 128, 64, 0.1, 1, None, 0, None)
    assert st != 0 and b"block table of 8 columns" in lib.sa_last_error()
    assert lib.sa_decode_workspace_bytes(2, 4, 128, 3) == 3 * 2 * 4 * 130 * 4
    assert lib.sa_decode_workspace_bytes(2, 4, 128, 1) == 0
    assert lib.sa_prefill_workspace_bytes() == 32            # counters and the status word (word 3)
    # the no-allocation decode refuses sizes past its scratch array before anything else (NULL tensors:
    # a call let through would stop at sa_decode's own NULL check, a different status)
    cap = int(lib.sa_decode_noalloc_scratch_bytes())
    B = cap // (16 * 32 * 130 * 4) + 1
    st = lib.sa_decode_noalloc(0, None, 4096, 128, None, None, 8192, 8192, 128, None, 256, 256, 1 << 20, None, 0,
                               None, 8 * 16, 16, None, 16, 2, 8, None, 4096, 128, B, 32, 8, 128, 64, 0.088, 16, None)
    assert st == -7 and b"scratch bytes" in lib.sa_last_error()
    # measurement aids: shapes checked before any launch
    assert lib.sa_mfma_rate(0, 10, None, 0, None) != 0 and b"per_cu 0" in lib.sa_last_error()
    assert lib.sa_mfma_rate(2, 10, None, 0, None) != 0 and b"NULL sink" in lib.sa_last_error()
    assert lib.sa_lds_read_rate(0, 0, None, 0, None) != 0 and b"iters 0" in lib.sa_last_error()
    # a sink shorter than one word per launched thread is refused before the launch
    assert lib.sa_mfma_rate(2, 10, fake, 1, None) != 0 and b"needs" in lib.sa_last_error()
    assert lib.sa_lds_read_rate(1, 10, fake, 1, None) != 0 and b"needs" in lib.sa_last_error()
    assert lib.sa_stage_rate(fake, 1024, 10, fake, 1 << 20, None) != 0 and b"needs 65536" in lib.sa_last_error()
    assert lib.sa_stage_rate(fake, 1 << 16, 10, fake, 1, None) != 0 and b"needs" in lib.sa_last_error()
    assert lib.sa_step_rate(3, fake, 1 << 16, 10, fake, 1 << 20, None) != 0 and b"layout 3" in lib.sa_last_error()
    assert lib.sa_step_rate(0, fake, 1024, 10, fake, 1 << 20, None) != 0 and b"needs 65536" in lib.sa_last_error()
    assert lib.sa_step_rate(1, fake, 1 << 16, 0, fake, 1 << 20, None) != 0 and b"steps 0" in lib.sa_last_error()
    assert lib.sa_step_rate(2, fake, 1 << 16, 10, fake, 1, None) != 0 and b"needs" in lib.sa_last_error()
    assert [lib.sa_step_rate_threads(k) for k in (0, 1, 2, 3)] == [512, 1024, 256, -1]
    # the timeline launch instruments only the persistent four-head kernel (workspace, four query heads
    # per CSR row, head dim 128) and refuses anything else, or a short record buffer, before any launch

    def timeline(D, ws, words, tl=fake, csr_rows=2):
        return lib.sa_prefill_timeline(0, fake, 8, 8, 8, fake, 8, 8, 8, fake, 8, 8, 8, fake, 8, 8, 8,
                                       fake, 8, fake, 8, csr_rows, 2, 1, 8, 2, 100, 100, D, 64, 0, 0.1,
                                       ws, 32 if ws else 0, tl, words, None)

    assert timeline(128, fake, 1 << 20, tl=None) == -6 and b"NULL timeline" in lib.sa_last_error()
    assert timeline(128, None, 1 << 20) == -2 and b"four-head" in lib.sa_last_error()
    assert timeline(64, fake, 1 << 20) == -2 and b"four-head" in lib.sa_last_error()
    assert timeline(128, fake, 1 << 20, csr_rows=8) == -2 and b"four-head" in lib.sa_last_error()
    assert timeline(128, fake, 35) == -7 and b"timeline of 35 words" in lib.sa_last_error()
    words = lib.sa_prefill_timeline_words(0)
    assert words > 0 and words % 36 == 0
    assert lib.sa_prefill_timeline_words(7) == -1


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setenv("SPARSE_ATTN_HIP_LIB", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(_lib.HipLibraryError):
        _lib.load()
