"""The worker benchmark with the reference's command line
(flexkv_amd/benchmarks/benchmark_workers.py): config parsing, the SSD
transfer types end to end through a spawned worker process (host code only),
and, on a GPU, H2D / D2H through a spawned GPU worker on both paths."""
import json

import pytest
import torch

from flexkv_amd.benchmarks import benchmark_workers as bw
from flexkv_amd.common.storage import KVCacheLayoutType
from flexkv_amd.common.transfer import TransferType


def _config(tmp_path, **cache):
    cfg = {
        "ModelConfig": {"num_layers": 4, "num_kv_heads": 2, "head_size": 64,
                        "dtype": "float16", "use_mla": False, "tp_size": 1, "dp_size": 1},
        "CacheConfig": {"tokens_per_block": 16, "cpu_kv_layout_type": "LAYERWISE",
                        "ssd_kv_layout_type": "LAYERWISE", "num_cpu_blocks": 64,
                        "num_ssd_blocks": 128, "use_pinned_memory": False,
                        "ssd_cache_dir": str(tmp_path / "ssd"),
                        # keys of parts this package does not have
                        "enable_remote": False, "remote_cache_path": None,
                        "enable_trace": False, "use_gds": False, **cache},
    }
    (tmp_path / "ssd").mkdir(exist_ok=True)
    p = tmp_path / "cfg.json"
    p.write_text(json.dumps(cfg))
    return str(p)


def test_example_config_parses():
    args = bw.parse_args(["--transfer-type", "D2H", "--num-blocks", "64"])
    model, cache, bench = bw.make_configs(args)
    assert model.dtype == torch.bfloat16 and model.num_layers == 32
    assert cache.cpu_kv_layout_type == KVCacheLayoutType.LAYERWISE
    assert not cache.use_ce_transfer_d2h and cache.transfer_sms_d2h == 8
    assert bench.transfer_type == TransferType.D2H and bench.num_blocks_to_transfer == 64


def _tp_config(tmp_path, tp=2, **cache):
    p = tmp_path / "tp.json"
    cfg = json.loads(open(_config(tmp_path, **cache)).read())
    cfg["ModelConfig"]["tp_size"] = tp
    p.write_text(json.dumps(cfg))
    return str(p)


def test_reference_style_keys_are_ignored_and_tp_accepted(tmp_path):
    args = bw.parse_args(["--config", _config(tmp_path)])
    model, cache, _ = bw.make_configs(args)
    assert model.dtype == torch.float16 and cache.num_ssd_blocks == 128
    model, _, _ = bw.make_configs(bw.parse_args(["--config", _tp_config(tmp_path)]))
    assert model.tp_size == 2


@pytest.mark.parametrize("kind,shuffle,entries", [("H2DISK", False, 0), ("DISK2H", True, 0),
                                                  ("DISK2H", False, 16)])
def test_ssd_benchmark_runs(tmp_path, kind, shuffle, entries):
    args = bw.parse_args(["--config", _config(tmp_path, ssd_cache_iouring_entries=entries),
                          "--transfer-type", kind, "--num-blocks", "24",
                          "--benchmark-round", "2"] + (["--shuffle-ids"] if shuffle else []))
    res = bw.bench_worker(args)
    # 24 blocks x 16 tokens x (4 layers x 2 heads x 64 x 2 (K,V) x 2 bytes)
    assert res["bytes"] == 24 * 16 * 4 * 2 * 64 * 2 * 2
    assert res["gb_per_s"] > 0 and res["path"] == "ssd"


def test_unsupported_transfer_type(tmp_path):
    with pytest.raises(ValueError, match="Unsupported transfer type"):
        bw.bench_worker(bw.parse_args(["--config", _config(tmp_path),
                                       "--transfer-type", "REMOTE2H"]))


def test_more_blocks_than_the_cache_holds(tmp_path):
    with pytest.raises(ValueError, match="exceeds"):
        bw.bench_worker(bw.parse_args(["--config", _config(tmp_path), "--transfer-type",
                                       "H2DISK", "--num-blocks", "65"]))


@pytest.mark.gpu
@pytest.mark.parametrize("kind,ce", [("D2H", False), ("H2D", False), ("D2H", True),
                                     ("H2D", True)])
def test_gpu_benchmark_runs(tmp_path, kind, ce):
    """H2D / D2H through a spawned GPUCPUTransferWorker fed TensorSharedHandles,
    on the zero-copy kernel and the copy-engine path."""
    cfg = _config(tmp_path, use_pinned_memory=True, use_ce_transfer_h2d=ce,
                  use_ce_transfer_d2h=ce)
    res = bw.bench_worker(bw.parse_args(["--config", cfg, "--transfer-type", kind,
                                         "--num-blocks", "48", "--shuffle-ids",
                                         "--benchmark-round", "3"]))
    assert res["bytes"] == 48 * 16 * 4 * 2 * 64 * 2 * 2
    assert res["path"] == ("ce" if ce else "kernel") and res["gb_per_s"] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("kind,ce", [("D2H", False), ("H2D", True)])
def test_gpu_benchmark_runs_tp(tmp_path, kind, ce):
    """tp_size = 2: a spawned tpGPUCPUTransferWorker over two ranks (each
    holding half the heads) on cuda:0; the op moves every rank's bytes."""
    cfg = _tp_config(tmp_path, use_pinned_memory=True, use_ce_transfer_h2d=ce,
                     use_ce_transfer_d2h=ce)
    res = bw.bench_worker(bw.parse_args(["--config", cfg, "--transfer-type", kind,
                                         "--num-blocks", "48", "--shuffle-ids",
                                         "--benchmark-round", "3"]))
    assert res["bytes"] == 48 * 16 * 4 * 2 * 64 * 2 * 2
    assert res["gb_per_s"] > 0


REFERENCE_CONFIG = "/root/reference/benchmarks/example_config.json"


@pytest.mark.skipif(not __import__("os").path.exists(REFERENCE_CONFIG),
                    reason="the reference tree is not present")
def test_reference_example_config_loads():
    """The reference's own benchmark config (read from the reference tree
    where it is present) loads: its remote, trace and GDS keys are dropped,
    layout names become layout types."""
    model, cache, bench = bw.make_configs(bw.parse_args(["--config", REFERENCE_CONFIG,
                                                         "--transfer-type", "D2H"]))
    assert model.num_layers > 0 and model.dtype in (torch.bfloat16, torch.float16)
    assert isinstance(cache.cpu_kv_layout_type, KVCacheLayoutType)
    assert bench.transfer_type == TransferType.D2H


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_bench_refuses_more_than_one_gpu(gpus):
    """bench.py measures one GPU; asked for more it exits with status 2 and
    says so, before touching any device."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", gpus],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_kernel_section_key_ignores_comments_only(tmp_path):
    """The counter profiles are keyed by the kernel section of kv_transfer.hip:
    a comment or blank-line change keeps the key, a code change (even inside
    a line that carries a comment) changes it, and text after the section's
    end does not count."""
    import os
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, root)
    import bench
    src = open(bench.KERNEL_SOURCE, "rb").read()
    end = src.find(bench.KERNEL_SECTION_END)
    assert end > 0
    base = bench.kernel_section_sha16()

    def key(data: bytes) -> str:
        p = tmp_path / "k.hip"
        p.write_bytes(data)
        return bench.kernel_section_sha16(str(p))

    assert key(src) == base
    assert key(b"// another comment\n\n" + src) == base
    assert key(src[:end].replace(b"\n", b"  // note\n", 1) + src[end:]) == base
    assert key(src[:end] + src[end:] + b"\nint tail_change;\n") == base
    assert key(b"#define FKV_EXTRA 1\n" + src) != base
    first_code = src.find(b"\n#include")
    assert first_code > 0
    assert key(src[:first_code] + b"\nint x;  // a comment\n" + src[first_code:]) != base
