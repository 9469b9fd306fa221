"""The committed measurement summaries name workloads that exist: every
workload name in profiles/*.md (table rows and `--config` arguments) is a
configuration of workloads.py, so each summary's command can be rerun as
written, and every profiles/traffic_<workload>.json (which bench.py reads for
roofline.traffic) belongs to a workload and matches its algorithmic bytes."""
import json
import re
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]
PREFIXES = ("cpu_ref_", "prefill_", "dsv3_", "decode_", "ue8m0_", "f16_", "bf16_r32_", "ref4_",
            "tp8_", "tp4_", "dsa_", "gemm_", "mla_")
NAME = re.compile(r"\b(?:%s)[a-z0-9_]*\d[a-z0-9_]*" % "|".join(PREFIXES))


def all_workloads():
    from fagq_mi355x import workloads as wl
    dicts = [wl.CONFIGS, wl.TYPED_CONFIGS, wl.REFERENCE_MODE_CONFIGS, wl.PARTS_CONFIGS,
             wl.DSA_CONFIGS, wl.GEMM_CONFIGS, wl.MLA_CONFIGS]
    names = [n for d in dicts for n in d]
    assert len(names) == len(set(names)), "a workload name is defined twice"
    return {n: w for d in dicts for n, w in d.items()}


def test_profiles_name_existing_workloads(pkg):
    known = all_workloads()
    seen = set()
    for md in sorted((REPO / "profiles").glob("*.md")):
        for name in NAME.findall(md.read_text()):
            seen.add(name)
            assert name in known, f"{md.name}: unknown workload {name}"
    assert "dsv3_16384x7168" in seen


def test_traffic_files_match_their_workloads(pkg):
    known = all_workloads()
    for f in sorted((REPO / "profiles").glob("traffic_*.json")):
        name = f.stem[len("traffic_"):]
        assert name in known, f"{f.name}: unknown workload"
        d = json.loads(f.read_text())
        assert d["workload"] == name, f.name
        assert abs(d["hbm_bytes_per_launch"] - d["fetch_bytes_per_launch"] -
                   d["write_bytes_per_launch"]) <= 1, f.name
        if "algorithmic_bytes" in d:        # HBM-bound kernels: traffic against the byte model
            try:
                model = known[name].algorithmic_bytes()
            except TypeError:               # DSA: the byte model needs the rows' valid blocks
                model = None
            if model is not None:
                assert d["algorithmic_bytes"] == model, f.name
            assert 0.9 < d["traffic_over_algorithmic"] < 1.2, f.name
            assert abs(d["hbm_bytes_per_launch"] / d["algorithmic_bytes"] -
                       d["traffic_over_algorithmic"]) < 1e-3, f.name
        else:                               # the GEMM: operand re-reads against the minimum
            assert abs(d["fetch_bytes_per_launch"] / d["min_read_bytes"] -
                       d["fetch_over_min_read"]) < 1e-2, f.name
            assert abs(d["write_bytes_per_launch"] / d["min_write_bytes"] -
                       d["write_over_min_write"]) < 1e-3, f.name
