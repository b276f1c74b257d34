"""bench.py's host-side contract, checked without a GPU: the one-GPU rule and
the rule that the HBM traffic figure is reported only while the decode kernel
sources are the ones the committed rocprofv3 counter summary measured."""

import importlib.util
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "--gpus 2 is not supported" in r.stderr and "one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line for a configuration that was not measured


def test_traffic_figure_follows_the_measured_sources():
    b = _bench()
    with open(os.path.join(ROOT, "profiles", "paged_decode_bf16_qwen3_0.6b_b64_pmc.json")) as f:
        rec = json.load(f)
    # the committed summary names the sources it measured and adds up
    assert rec["hbm_bytes_per_launch"] == rec["split_kernel_bytes"] + rec["merge_kernel_bytes"]
    kib = 1024
    split = rec["fetch_kib_split"] * kib * rec["fetch_scale"] + rec["write_kib_split"] * kib * rec["write_scale"]
    merge = rec["fetch_kib_merge"] * kib * rec["fetch_scale"] + rec["write_kib_merge"] * kib * rec["write_scale"]
    assert abs(split - rec["split_kernel_bytes"]) <= kib and abs(merge - rec["merge_kernel_bytes"]) <= kib
    traffic, source = b.pmc_traffic("paged_decode_bf16_qwen3_0.6b_b64", b.DECODE_SOURCES)
    if rec["sources_sha16"] == b.sources_sha16(b.DECODE_SOURCES):
        assert traffic == rec["hbm_bytes_per_launch"] and rec["sources_sha16"] in source
    else:
        assert traffic is None and source.startswith("stale")
    # any other source set (here: the prefill kernel as well) reads as stale
    other = b.DECODE_SOURCES + ("csrc/paged_prefill.hip",)
    traffic, source = b.pmc_traffic("paged_decode_bf16_qwen3_0.6b_b64", other)
    assert traffic is None and source.startswith("stale")
    traffic, source = b.pmc_traffic("no_such_kernel", b.DECODE_SOURCES)
    assert traffic is None and "no committed" in source
