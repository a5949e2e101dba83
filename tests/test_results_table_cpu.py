"""profiles/results.md is what the table writer makes of profiles/results.json
(the bench line it was generated from), so the committed table cannot drift
from its source."""
import os

from flexkv_amd.benchmarks import results_table

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_results_table_matches_its_source():
    src = os.path.join(ROOT, "profiles", "results.json")
    with open(os.path.join(ROOT, "profiles", "results.md")) as fh:
        committed = fh.read()
    assert results_table.table(results_table.load(src), "one MI355X") == committed


def test_results_table_reads_bench_output(tmp_path):
    src = os.path.join(ROOT, "profiles", "results.json")
    p = results_table.load(src)
    import json
    log = tmp_path / "bench.log"
    log.write_text("warming up\n" + json.dumps(p) + "\n")
    assert results_table.load(str(log)) == p
