"""bench.py's profile stamp: every summary under profiles/ records a digest
of the kernel sources it was taken on, and the bench line marks the
headline's roofline stale when the tree's sources differ.  CPU only."""
import json
import os

import pytest

from conftest import ROOT


@pytest.fixture(scope="module")
def bench():
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_digest_covers_every_kernel_source_and_the_build_flags(bench):
    files = [os.path.relpath(f, ROOT) for f in bench.kernel_source_files()]
    assert "breeze-engine_amd/breeze_amd/_build.py" in files
    for name in ("qmm.hip", "qmm_common.h", "dec_kernel.h", "dec8_kernel.h", "prefill_kernel.h"):
        assert f"breeze-engine_amd/csrc/{name}" in files


def test_digest_follows_content(bench, tmp_path):
    a, b = tmp_path / "a.hip", tmp_path / "b.h"
    a.write_text("kernel one\n")
    b.write_text("header\n")
    d0 = bench.kernel_sources_digest([str(a), str(b)])
    assert d0 == bench.kernel_sources_digest([str(a), str(b)])
    a.write_text("kernel two\n")
    assert bench.kernel_sources_digest([str(a), str(b)]) != d0


def test_traffic_record_is_stale_unless_its_digest_is_the_trees(bench, tmp_path):
    p = tmp_path / "traffic.json"
    rec = {"bytes_per_launch": 1, "sources_digest": bench.kernel_sources_digest()}
    p.write_text(json.dumps(rec))
    assert bench.traffic_record(str(p)) == (rec, False)
    rec["sources_digest"] = "0" * 16
    p.write_text(json.dumps(rec))
    assert bench.traffic_record(str(p))[1] is True
    del rec["sources_digest"]
    p.write_text(json.dumps(rec))
    assert bench.traffic_record(str(p))[1] is True
    assert bench.traffic_record(str(tmp_path / "missing.json")) == (None, True)


def test_every_kernel_summary_carries_a_digest():
    for f in sorted(os.listdir(os.path.join(ROOT, "profiles"))):
        if f.endswith(".txt"):
            text = open(os.path.join(ROOT, "profiles", f)).read()
            assert "Kernel sources digest" in text, f
