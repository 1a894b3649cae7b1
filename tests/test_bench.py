"""bench.py's host-side logic (CPU): the NS kernel family named in the
roofline for each tile geometry, and the single-GPU guard."""

from __future__ import annotations

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_ns_family_follows_the_library_dispatch():
    # LDS-resident kernel: mp == 128 and np in {128, 256, 512}
    assert bench.ns_family(128, 128) == "lds"
    assert bench.ns_family(128, 256) == "lds"
    assert bench.ns_family(128, 512) == "lds"
    assert bench.ns_family(128, 384) == "small" and bench.ns_family(128, 1024) == "small"
    # 512 x 512: Gram kernel + fused GramB/Apply; the three products with "stream3"
    assert bench.ns_family(512, 512) == "fused"
    assert bench.ns_family(512, 512, "stream3") == "stream"
    # streamed 256-blocks: both padded edges multiples of 256
    assert bench.ns_family(256, 1024) == "stream"
    assert bench.ns_family(1024, 3072) == "stream"
    # everything else: 128-block kernels
    assert bench.ns_family(128, 384) == "small"
    assert bench.ns_family(640, 768) == "small"
    assert bench.ns_family(384, 384) == "small"
    assert bench.ns_family(512, 512, "block128") == "small"
    # operands with at most 64 real rows in a 128-row buffer: their own rows in LDS
    assert bench.ns_family(128, 1024, rows=16) == "few_rows" and bench.ns_family(128, 2048, rows=16) == "few_rows"
    assert bench.ns_family(128, 1024, rows=32) == "few_rows" and bench.ns_family(128, 2048, rows=32) == "small"
    assert bench.ns_family(128, 128, rows=64) == "few_rows" and bench.ns_family(128, 512, rows=64) == "lds"
    assert bench.ns_family(128, 1024, rows=64) == "small" and bench.ns_family(128, 384, rows=40) == "small"
    assert bench.ns_family(128, 384, rows=20) == "few_rows" and bench.ns_family(128, 128, rows=100) == "lds"
    assert bench.ns_family(128, 1024, "block128", rows=16) == "small"
    assert set(bench.NS_KERNELS) == {"fused", "stream", "lds", "small", "few_rows"}


def test_few_rows_rule_matches_the_binding():
    from himuon_amd import _native as nat

    for m in (1, 16, 17, 32, 33, 48, 64, 65, 128):
        for np_ in (128, 256, 384, 512, 640, 768, 1024, 1536, 2048, 4096):
            expect = nat.few_rows_supported(m, 128, np_)
            assert (bench.ns_family(128, np_, rows=m) == "few_rows") == expect, (m, np_)
    assert not nat.few_rows_supported(16, 256, 1024)


def test_ns_flops_is_the_normative_count():
    # 5 (4 m^2 n + 2 m^3), m <= n: 30 T^3 for a square tile
    assert bench.ns_flops(512, 512) == 30 * 512**3
    assert bench.ns_flops(128, 128) == 30 * 128**3
    assert bench.ns_flops(1024, 2048) == 5 * (4 * 1024**2 * 2048 + 2 * 1024**3)


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_cpu_baseline_times_a_whole_layer_and_extrapolates():
    import torch

    r = bench.cpu_baseline(3, [(600, 700), (256, 300), (100, 90)], 256, torch.bfloat16, budget_s=2.0)
    assert r["kind"] == "port" and r["cores"] >= 1
    assert "full layers" in r["sample"] and "x3 extrapolated" in r["unit"]
    assert abs(r["value"] - 3 * r["layer_ms"]) <= 0.2
    assert r["cpu"]


def test_reference_microbenchmark_points():
    # exp_ns5_rect_bench.py:83-103: M <= N from DIMS with M N + 2 M^2 <= 49152 -> 19 shapes
    shapes = bench.rect_shapes()
    assert len(shapes) == 19 and (128, 128) in shapes and (16, 2048) in shapes and (64, 1024) not in shapes
    assert all(m <= n and m * n + 2 * m * m <= 49152 for m, n in shapes)
    # exp_ns_kernel_microbench.py:279: B = 32, 128, 512, 2048 at T = 128, each with a reference
    # figure; B = 65,536 (the cfg5 sub-batch) is this build's addition and has none
    assert sorted(bench.NS_MICRO_B.values()) == [32, 128, 512, 2048, 65536]
    assert set(bench.NS_MICRO_REF_MS) == {32, 128, 512, 2048}


def test_tile_elements_counts_covered_parameter_elements():
    from types import SimpleNamespace

    shapes = [(300, 200), (128, 128), (77, 130)]
    th = tw = 128
    counts = [(-(-h // th)) * (-(-w // tw)) for h, w in shapes]
    tile0 = [sum(counts[:i]) for i in range(len(counts))]
    grp = SimpleNamespace(params=[SimpleNamespace(shape=s) for s in shapes], tile0=tile0, tile_counts=counts,
                          tile_h=th, tile_w=tw)
    n_all = sum(counts)
    assert bench._tile_elements(grp, n_all) == sum(h * w for h, w in shapes)
    # the first tile row of the 300 x 200 matrix: 128 x 128 + 128 x 72
    assert bench._tile_elements(grp, 2) == 128 * 128 + 128 * 72
    assert bench._tile_elements(grp, 0) == 0
