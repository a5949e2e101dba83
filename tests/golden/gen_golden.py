"""Writes the committed fixtures in this directory.

    python tests/golden/gen_golden.py

tiny_vectors.npz: tiny transfers with explicit inputs and outputs.  Expected
  host caches come from an element-by-element loop over shaped arrays and
  expected GPU layers from numpy indexing (tests/kvcase.py), not from the
  oracle; the script also checks the oracle agrees before writing.
config0_digests.json: SHA-256 digests for the CPU-plumbing configuration
  (4 layers, fp16 K/V [256,16,8,128], block-wise host [512,4,2,16,8,128],
  64 distinct random ids, seed 1000), inputs from oracle/inputs.py.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.dirname(HERE)):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import inputs  # noqa: E402
from kvcase import KVCase, brute_force_d2h  # noqa: E402

CONFIG0_SEED = 1000
TINY_SHAPES = [
    dict(layers_total=3, num_layers=2, start_layer=1, kv=2, ng=5, nh=7, tokens=2, heads=2, dim=4),
    dict(layers_total=3, num_layers=3, start_layer=0, kv=1, ng=4, nh=6, tokens=2, heads=1, dim=8,
         layout="LAYERWISE"),
    dict(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=4, nh=5, tokens=1, heads=2, dim=8,
         tp=2, rank=1),
]
TINY_IDS = [([3, 0, 2], [1, 4, 3]), ([1, 3], [5, 0]), ([0, 2, 3], [4, 1, 2])]


def config0_case() -> KVCase:
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=256, nh=512, tokens=16,
                  heads=8, dim=128, dtype=np.uint16)
    n = int(np.prod(case.gpu_shape()))
    case.gpu = [inputs.normal_bits(CONFIG0_SEED, n, "fp16", offset=l * n).reshape(case.gpu_shape())
                for l in range(4)]
    case.host = np.full(case.host_shape(), 0x5A5A, dtype=np.uint16)
    return case


def config0_ids():
    return (inputs.distinct_ids(CONFIG0_SEED * 7 + 1, 64, 256),
            inputs.distinct_ids(CONFIG0_SEED * 7 + 2, 64, 512))


def main() -> None:
    import oracle

    arrays = {}
    meta = []
    for i, (shape, (g, c)) in enumerate(zip(TINY_SHAPES, TINY_IDS)):
        case = KVCase(**shape).fill(seed=100 + i)
        gids, cids = np.array(g, np.int64), np.array(c, np.int64)
        want_host = brute_force_d2h(case, gids, cids)
        s = case.strides()
        chk = case.host.copy()
        oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], cids, chk,
                                  s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"],
                                  case.start_layer, False, is_mla=case.kv == 1,
                                  cpu_startoff_inside_chunks=s["startoff"])
        assert np.array_equal(chk, want_host), f"oracle disagrees on tiny case {i}"
        case_after = KVCase(**shape)
        case_after.host = want_host
        want_gpu = case_after.expect_h2d(gids, cids, [np.zeros_like(x) for x in case.gpu])
        arrays[f"c{i}_host"] = case.host
        arrays[f"c{i}_gids"] = gids
        arrays[f"c{i}_cids"] = cids
        arrays[f"c{i}_want_host"] = want_host
        for l, x in enumerate(case.gpu):
            arrays[f"c{i}_gpu{l}"] = x
            arrays[f"c{i}_want_gpu{l}"] = want_gpu[l]
        meta.append({"shape": shape})
    arrays["meta"] = np.array(json.dumps(meta))
    np.savez_compressed(os.path.join(HERE, "tiny_vectors.npz"), **arrays)

    case = config0_case()
    gids, cids = config0_ids()
    want_host = case.expect_d2h(gids, cids)
    s = case.strides()
    host = case.host.copy()
    oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], cids, host,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"], 0, False)
    assert np.array_equal(host, want_host), "oracle disagrees with indexing on config 0"
    case.host = host
    back = case.expect_h2d(gids, cids, [np.zeros_like(x) for x in case.gpu])
    digests = {
        "config": "4 layers, fp16 K/V [256,16,8,128] -> blockwise host [512,4,2,16,8,128], "
                  "64 distinct ids, host initialised to 0x5A5A, H2D into zeroed GPU layers",
        "seed": CONFIG0_SEED,
        "gpu_ids_head": gids[:8].tolist(),
        "cpu_ids_head": cids[:8].tolist(),
        "gpu_input_sha256": hashlib.sha256(b"".join(x.tobytes() for x in case.gpu)).hexdigest(),
        "d2h_host_sha256": hashlib.sha256(host.tobytes()).hexdigest(),
        "h2d_gpu_sha256": hashlib.sha256(b"".join(x.tobytes() for x in back)).hexdigest(),
    }
    with open(os.path.join(HERE, "config0_digests.json"), "w") as fh:
        json.dump(digests, fh, indent=2)
        fh.write("\n")
    print("wrote tiny_vectors.npz and config0_digests.json")


if __name__ == "__main__":
    main()
