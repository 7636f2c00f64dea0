"""The task-queue consumer of the gpu_workload harness (switch-l4t-gpu_amd/task_unit.py;
contract of deploy/cluster/gpu_task_example.py:21-128) on canned harness reports -- good,
truncated, WRONG, done:false, missing sizes, out-of-bounds numbers, the legacy text form --
and through fake harness programs for the subprocess flow (CPU); on the GPU, the live
`gpu_workload --json` report."""
import json
import os
import stat

import pytest

import task_unit as tu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def report(**over):
    """A gfx950 `gpu_workload --json` report in the harness's schema (numbers of an MI355X run)."""
    d = {"ptx": "build/switch_gpu.co",
         "kernels": {"sgemm": "CORRECT", "sgemm_naive": "CORRECT", "sgemm_tiled4": "CORRECT", "sgemm_opt": "CORRECT"},
         "sgemm": [{"n": 256, "ms": 0.0, "gflops": 4300.2, "us": 7.8}, {"n": 512, "ms": 0.0, "gflops": 21000.5, "us": 12.8},
                   {"n": 1024, "ms": 0.0, "gflops": 79000.0, "us": 27.2}],
         "sgemm4": [{"n": 256, "ms": 0.0, "gflops": 3000.0, "us": 11.2}, {"n": 512, "ms": 0.0, "gflops": 15000.0, "us": 17.9},
                    {"n": 1024, "ms": 0.1, "gflops": 60000.0, "us": 35.8}],
         "membw_gbps": 6712.4, "membw_mb": 1024, "arch": "gfx950", "device": "AMD gfx950 GPU, 256 CUs", "done": True}
    d.update(over)
    return json.dumps(d)


TEGRA_JSON = json.dumps({"ptx": "switch_gpu_native.ptx",
                         "kernels": {"sgemm": "CORRECT", "sgemm_naive": "CORRECT", "sgemm_tiled4": "CORRECT"},
                         "sgemm": [{"n": 256, "ms": 1.0, "gflops": 57.6}, {"n": 512, "ms": 4.2, "gflops": 63.6},
                                   {"n": 1024, "ms": 33.2, "gflops": 64.6}],
                         "sgemm4": [{"n": 256, "ms": 0.5, "gflops": 65.5}, {"n": 512, "ms": 3.5, "gflops": 76.8},
                                    {"n": 1024, "ms": 23.2, "gflops": 92.7}],
                         "membw_gbps": 22.3, "done": True})

TEXT = """device: AMD gfx950 GPU, 256 CUs
sgemm 256: CORRECT
sgemm_naive 256: CORRECT
sgemm 256x256x256: 0.008 ms/iter, 4300.2 GFLOPS
sgemm_tiled4 256: CORRECT
sgemm4 256x256x256: 0.011 ms/iter, 3000.0 GFLOPS
sgemm 512x512x512: 0.013 ms/iter, 21000.5 GFLOPS
sgemm 1024x1024x1024: 0.027 ms/iter, 79000.0 GFLOPS
membw read (1024MB x10): 1.6000 s, 6712.4 GB/s
WORKLOAD_DONE
"""


def test_good_report_accepted_and_reverified():
    r = tu.parse_json(report())
    assert r["correct"] is True and r["arch"] == "gfx950"
    assert r["gflops"] == {"256": 4300.2, "512": 21000.5, "1024": 79000.0} and r["gbps"] == 6712.4
    tu.verify_unit(r)                                     # the coordinator's re-check passes
    tu.verify_unit(json.loads(json.dumps(r)))             # also after a JSON round trip


def test_mi355x_numbers_fail_the_reference_tegra_bounds():
    """The reference's fixed (1, 1000) gates reject every MI355X result; the device bounds do not."""
    r = tu.parse_json(report())
    with pytest.raises(tu.UnitError, match="outside the sanity bounds"):
        tu.check_numbers(r["gflops"], r["gbps"], None)


def test_tegra_report_keeps_reference_bounds():
    r = tu.parse_json(TEGRA_JSON)
    assert r["arch"] is None and r["gflops"]["1024"] == 64.6
    tu.verify_unit(r)
    bad = json.loads(TEGRA_JSON)
    bad["sgemm"][2]["gflops"] = 4000.0                    # impossible on a Tegra X1
    with pytest.raises(tu.UnitError, match=r"gflops\[1024\]"):
        tu.parse_json(json.dumps(bad))


@pytest.mark.parametrize("cut", [1, 40, 200, -2])
def test_truncated_json_rejected(cut):
    with pytest.raises(tu.UnitError, match="unreadable|incomplete"):
        tu.parse_json(report()[:cut])


def test_done_false_or_missing_rejected():
    with pytest.raises(tu.UnitError, match="done flag"):
        tu.parse_json(report(done=False))
    d = json.loads(report())
    del d["done"]
    with pytest.raises(tu.UnitError, match="done flag"):
        tu.parse_json(json.dumps(d))


@pytest.mark.parametrize("kernel", ["sgemm", "sgemm_naive", "sgemm_opt"])
def test_wrong_verdict_rejected(kernel):
    d = json.loads(report())
    d["kernels"][kernel] = "WRONG"
    with pytest.raises(tu.UnitError, match=kernel):
        tu.parse_json(json.dumps(d))


def test_missing_sgemm_verdict_rejected():
    d = json.loads(report())
    del d["kernels"]["sgemm"]
    with pytest.raises(tu.UnitError, match="no sgemm verdict"):
        tu.parse_json(json.dumps(d))


def test_wrong_extra_shape_rejected():
    extra = [{"kernel": "sgemm_tiled", "m": 1023, "n": 1025, "k": 997, "verdict": "WRONG", "ms": 0.03, "gflops": 6e4}]
    with pytest.raises(tu.UnitError, match="sgemm_extra"):
        tu.parse_json(report(sgemm_extra=extra))


@pytest.mark.parametrize("size", [256, 512, 1024])
def test_missing_size_rejected(size):
    d = json.loads(report())
    d["sgemm"] = [r for r in d["sgemm"] if r["n"] != size]
    with pytest.raises(tu.UnitError, match=f"'{size}'"):
        tu.parse_json(json.dumps(d))


@pytest.mark.parametrize("field,value", [("gflops", 0.0), ("gflops", 2.0e5), ("gflops", None), ("gbps", 0.5),
                                         ("gbps", 9000.0), ("gbps", None)])
def test_out_of_bounds_numbers_rejected(field, value):
    d = json.loads(report())
    if field == "gflops":
        d["sgemm"][1]["gflops"] = value
    else:
        d["membw_gbps"] = value
    with pytest.raises(tu.UnitError):
        tu.parse_json(json.dumps(d))


def test_mall_sized_probe_gets_mall_bounds():
    """A probe buffer that fits the 256 MB MALL may read faster than HBM; past 512 MB it may not."""
    tu.parse_json(report(membw_gbps=12000.0, membw_mb=64))
    with pytest.raises(tu.UnitError, match="membw"):
        tu.parse_json(report(membw_gbps=12000.0, membw_mb=1024))


def test_unknown_device_rejected():
    with pytest.raises(tu.UnitError, match="no sanity bounds"):
        tu.parse_json(report(arch="gfx9999"))


def test_text_report():
    r = tu.parse_text(TEXT, arch="gfx950")
    assert r["kernels_verified"] == ["sgemm", "sgemm_naive", "sgemm_tiled4"] and r["membw_mb"] == 1024
    with pytest.raises(tu.UnitError, match="WORKLOAD_DONE"):
        tu.parse_text(TEXT.replace("WORKLOAD_DONE\n", ""), arch="gfx950")
    with pytest.raises(tu.UnitError, match="golden"):
        tu.parse_text(TEXT.replace("sgemm_naive 256: CORRECT", "sgemm_naive 256: WRONG"), arch="gfx950")
    with pytest.raises(tu.UnitError, match="1024"):
        tu.parse_text(TEXT.replace("sgemm 1024x1024x1024", "sgemm 1024x1024x1000"), arch="gfx950")
    with pytest.raises(tu.UnitError, match="membw"):
        tu.parse_text(TEXT.replace("membw read", "membw_read"), arch="gfx950")


def test_verify_unit_rejects_unverified_results():
    r = tu.parse_json(report())
    with pytest.raises(tu.UnitError, match="correct"):
        tu.verify_unit({**r, "correct": False})
    with pytest.raises(tu.UnitError, match="1024"):
        tu.verify_unit({**r, "gflops": {"256": 1.0e3, "512": 2.0e3}})


def fake_harness(tmp_path, script):
    p = tmp_path / "gpu_workload"
    p.write_text("#!/bin/bash\n" + script)
    p.chmod(p.stat().st_mode | stat.S_IXUSR)
    return str(p)


def test_run_unit_json(tmp_path):
    out = tmp_path / "out.json"
    out.write_text(report() + "\n")
    h = fake_harness(tmp_path, f'[ "$1" = --json ] || exit 9\ncat {out}\n')
    assert tu.run_unit(h, "x.co")["gflops"]["1024"] == 79000.0


def test_run_unit_falls_back_to_text(tmp_path):
    """A harness without --json reads the flag as its code-object path and fails; the unit
    re-runs it without the flag and reads the text lines."""
    out = tmp_path / "out.txt"
    out.write_text(TEXT)
    h = fake_harness(tmp_path, f'[ "$1" = --json ] && {{ echo "cannot open --json" >&2; exit 1; }}\ncat {out}\n')
    assert tu.run_unit(h, "x.co", arch="gfx950")["gbps"] == 6712.4


def test_run_unit_failures(tmp_path):
    with pytest.raises(tu.UnitError, match="exited 3"):
        tu.run_unit(fake_harness(tmp_path, 'echo "{\\"done\\":false}"; echo boom >&2; exit 3\n'), "x.co")
    with pytest.raises(tu.UnitError, match="timed out"):
        tu.run_unit(fake_harness(tmp_path, "sleep 5\n"), "x.co", timeout=0.5)
    with pytest.raises(tu.UnitError, match="cannot run"):
        tu.run_unit(str(tmp_path / "missing"), "x.co")


@pytest.mark.gpu
def test_live_harness_report(gpu):
    """The real harness on the GPU: its --json report passes the MI355X bounds."""
    binary = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "gpu_workload")
    co = os.path.join(ROOT, "switch-l4t-gpu_amd", "build", "switch_gpu.co")
    r = tu.run_unit(binary, co, timeout=120)
    print("unit result", json.dumps(r), flush=True)
    assert r["correct"] and r["arch"] == "gfx950" and r["membw_mb"] >= tu.MALL_MB
    assert set(r["kernels_verified"]) == {"sgemm", "sgemm_naive", "sgemm_tiled4", "sgemm_opt"}
    tu.verify_unit(r)
