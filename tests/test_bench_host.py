"""Host logic of bench.py (no GPU): traffic figures keyed by the kernel source they were measured on,
the rotation of independent inputs, and the one-GPU refusal."""
import hashlib
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def _fake_tree(tmp_path, prefill_src: bytes, measured_src: bytes) -> Path:
    csrc = tmp_path / "sparseattentioninfer_amd" / "csrc"
    csrc.mkdir(parents=True)
    (csrc / "prefill.hip").write_bytes(prefill_src)
    (csrc / "decode.hip").write_bytes(b"decode v1")
    prof = tmp_path / "profiles"
    prof.mkdir()
    entry = lambda src, name, n: {"kernel_source": name, "kernel_source_sha1": hashlib.sha1(src).hexdigest(),
                                  "summary": "profiles/t.md", "hbm_bytes_per_launch": n}
    (prof / "traffic.json").write_text(json.dumps({
        "prefill_cfg2": entry(measured_src, "prefill.hip", 111),
        "prefill_cfg1": entry(measured_src, "prefill.hip", 222),
        "decode_cfg3": entry(b"decode v1", "decode.hip", 333),
        "decode_cfg3_22": entry(b"decode v1", "decode.hip", 444),
    }))
    return tmp_path


def _line():
    roof = lambda: {"traffic": None}
    return {"roofline": roof(), "configs1": {"roofline": roof()},
            "decode": {"roofline": roof(), "at_22_blocks": {"kernel_us": 1.0}}}


def test_traffic_attached_only_for_the_source_it_was_measured_on(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "ROOT", _fake_tree(tmp_path, b"prefill v2", b"prefill v1"))
    line = _line()
    bench._attach_traffic(line, prefill_first=True)
    # prefill.hip changed after its counters were taken: null, with the reason
    assert line["roofline"]["traffic"] is None and "older prefill.hip" in line["roofline"]["traffic_source"]
    assert line["configs1"]["roofline"]["traffic"] is None
    # decode.hip is the measured source: the figures are attached and labelled as not measured here
    assert line["decode"]["roofline"]["traffic"] == 333
    assert line["decode"]["at_22_blocks"]["traffic"] == 444
    assert "not measured in this run" in line["decode"]["roofline"]["traffic_source"]


def test_traffic_attached_when_sources_match(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "ROOT", _fake_tree(tmp_path, b"prefill v1", b"prefill v1"))
    line = _line()
    bench._attach_traffic(line, prefill_first=True)
    assert line["roofline"]["traffic"] == 111 and line["configs1"]["roofline"]["traffic"] == 222


def test_decode_only_line_takes_the_decode_figure(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "ROOT", _fake_tree(tmp_path, b"prefill v1", b"prefill v1"))
    line = {"roofline": {"traffic": None}, "decode": {"roofline": {"traffic": None}}}
    bench._attach_traffic(line, prefill_first=False)
    assert line["roofline"]["traffic"] == 333


def test_committed_traffic_table_names_existing_sources():
    table = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    for key in ("prefill_cfg2", "prefill_cfg1", "decode_cfg3", "decode_cfg3_22"):
        e = table[key]
        assert (ROOT / "sparseattentioninfer_amd" / "csrc" / e["kernel_source"]).exists()
        assert e["hbm_bytes_per_launch"] == e["fetch_bytes_per_launch"] + e["write_bytes_per_launch"] > 0
        assert len(e["kernel_source_sha1"]) == 40


def test_rotation_launches_in_turn():
    calls = []
    rot = bench._rotation([lambda i=i: calls.append(i) for i in range(3)])
    for _ in range(7):
        rot()
    assert calls == [0, 1, 2, 0, 1, 2, 0]


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_more_than_one_gpu_is_refused(gpus):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", gpus], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU only" in r.stderr
