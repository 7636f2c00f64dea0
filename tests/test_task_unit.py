"""The task-queue consumer of the gpu_workload harness (switch-l4t-gpu_amd/task_unit.py; the
contract of deploy/cluster/gpu_task_example.py:21-24,57-102) on canned harness reports --
good, truncated, WRONG, done:false, missing sizes, out-of-bounds numbers, the text form -- and
through fake harness programs for the subprocess flow and the home lookup (CPU); on the GPU,
the live `gpu_workload --json` report."""
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


def accept_json(text):
    return tu.accept(tu.Report.from_json(text))


TEGRA_JSON = json.dumps({"ptx": "switch_gpu_native.ptx",
                         "kernels": {"sgemm": "CORRECT", "sgemm_naive": "CORRECT", "sgemm_tiled4": "CORRECT"},
                         "sgemm": [{"n": 256, "ms": 1.0, "gflops": 57.6}, {"n": 512, "ms": 4.2, "gflops": 63.6},
                                   {"n": 1024, "ms": 33.2, "gflops": 64.6}],
                         "sgemm4": [{"n": 256, "ms": 0.5, "gflops": 65.5}, {"n": 512, "ms": 3.5, "gflops": 76.8},
                                    {"n": 1024, "ms": 23.2, "gflops": 92.7}],
                         "membw_gbps": 22.3, "done": True})

TEXT = """device: AMD Instinct MI355X, 256 CUs (gfx950)
sgemm 256: CORRECT
sgemm_naive 256: CORRECT (0 bad cells)
sgemm 256x256x256: 0.008 ms/iter, 4300.2 GFLOPS
sgemm_tiled4 256: CORRECT
sgemm4 256x256x256: 0.011 ms/iter, 3000.0 GFLOPS
sgemm 512x512x512: 0.013 ms/iter, 21000.5 GFLOPS
sgemm 1024x1024x1024: 0.027 ms/iter, 79000.0 GFLOPS
membw read (1024MB x10): 1.6000 s, 6712.4 GB/s
WORKLOAD_DONE
"""


def test_good_report_accepted_and_rechecked():
    r = accept_json(report())
    assert r["correct"] is True and r["arch"] == "gfx950"
    assert r["gflops"] == {"256": 4300.2, "512": 21000.5, "1024": 79000.0} and r["gbps"] == 6712.4
    tu.recheck(r)                                         # the coordinator's re-check passes
    tu.recheck(json.loads(json.dumps(r)))                 # also after a JSON round trip


def test_mi355x_numbers_fail_the_reference_tegra_bounds():
    """The reference's fixed (1, 1000) gates reject every MI355X result; the device limits do not."""
    rep = tu.Report.from_json(report())
    rep.arch = None
    findings = tu.audit(rep)
    assert len(findings) == 4 and all("outside the sanity bounds" in f for f in findings)


def test_tegra_report_keeps_reference_bounds():
    r = accept_json(TEGRA_JSON)
    assert r["arch"] is None and r["gflops"]["1024"] == 64.6
    tu.recheck(r)
    bad = json.loads(TEGRA_JSON)
    bad["sgemm"][2]["gflops"] = 4000.0                    # impossible on a Tegra X1
    with pytest.raises(tu.Rejected, match=r"n = 1024: 4000.0 GFLOPS"):
        accept_json(json.dumps(bad))


@pytest.mark.parametrize("cut", [1, 40, 200, -2])
def test_truncated_json_rejected(cut):
    with pytest.raises(tu.Rejected, match="unreadable|incomplete"):
        accept_json(report()[:cut])


def test_done_false_or_missing_rejected():
    with pytest.raises(tu.Rejected, match="done flag"):
        accept_json(report(done=False))
    d = json.loads(report())
    del d["done"]
    with pytest.raises(tu.Rejected, match="done flag"):
        accept_json(json.dumps(d))


@pytest.mark.parametrize("kernel", ["sgemm", "sgemm_naive", "sgemm_opt"])
def test_wrong_verdict_rejected(kernel):
    d = json.loads(report())
    d["kernels"][kernel] = "WRONG"
    with pytest.raises(tu.Rejected, match=f"golden check: {kernel}"):
        accept_json(json.dumps(d))


def test_missing_sgemm_verdict_rejected():
    d = json.loads(report())
    del d["kernels"]["sgemm"]
    with pytest.raises(tu.Rejected, match="no sgemm verdict"):
        accept_json(json.dumps(d))


def test_wrong_extra_shape_rejected():
    extra = [{"kernel": "sgemm_tiled", "m": 1023, "n": 1025, "k": 997, "verdict": "WRONG", "ms": 0.03, "gflops": 6e4}]
    with pytest.raises(tu.Rejected, match="sgemm_extra:sgemm_tiled:1023x1025x997"):
        accept_json(report(sgemm_extra=extra))
    ok = [dict(extra[0], verdict="CORRECT")]
    assert accept_json(report(sgemm_extra=ok))["kernels_verified"] == ["sgemm", "sgemm_naive", "sgemm_opt",
                                                                         "sgemm_tiled4"]


@pytest.mark.parametrize("size", [256, 512, 1024])
def test_missing_size_rejected(size):
    d = json.loads(report())
    d["sgemm"] = [r for r in d["sgemm"] if r["n"] != size]
    with pytest.raises(tu.Rejected, match=f"no SGEMM timing at n = {size}"):
        accept_json(json.dumps(d))


@pytest.mark.parametrize("field,value", [("gflops", 0.0), ("gflops", 2.0e5), ("gflops", None), ("gbps", 0.5),
                                         ("gbps", 9000.0), ("gbps", None), ("gbps", True)])
def test_out_of_bounds_numbers_rejected(field, value):
    d = json.loads(report())
    if field == "gflops":
        d["sgemm"][1]["gflops"] = value
    else:
        d["membw_gbps"] = value
    with pytest.raises(tu.Rejected, match="n = 512" if field == "gflops" else "membw"):
        accept_json(json.dumps(d))


def test_mall_sized_probe_gets_mall_bounds():
    """A probe buffer that fits the 256 MB MALL may read faster than HBM; past 512 MB it may not."""
    accept_json(report(membw_gbps=12000.0, membw_mb=64))
    with pytest.raises(tu.Rejected, match="membw"):
        accept_json(report(membw_gbps=12000.0, membw_mb=1024))


def test_unknown_device_rejected():
    with pytest.raises(tu.Rejected, match="no sanity bounds for device 'gfx9999'"):
        accept_json(report(arch="gfx9999"))


def test_every_finding_reported_at_once():
    d = json.loads(report(done=False, membw_gbps=None))
    d["kernels"]["sgemm_opt"] = "WRONG"
    d["sgemm"] = d["sgemm"][:1]
    with pytest.raises(tu.Rejected) as exc:
        accept_json(json.dumps(d))
    f = exc.value.findings
    assert len(f) == 5, f
    assert "done flag" in f[0] and "sgemm_opt" in f[1] and "n = 512" in f[2] and "n = 1024" in f[3] and "membw" in f[4]


def test_text_report():
    rep = tu.Report.read(TEXT)
    assert rep.form == "text" and rep.arch == "gfx950"          # read from the device line
    r = tu.accept(rep)
    assert r["kernels_verified"] == ["sgemm", "sgemm_naive", "sgemm_tiled4"] and r["membw_mb"] == 1024
    assert r["gflops"] == {"256": 4300.2, "512": 21000.5, "1024": 79000.0}
    no_device = TEXT.split("\n", 1)[1]
    assert tu.Report.read(no_device).arch is None and tu.Report.read(no_device, "gfx950").arch == "gfx950"
    with pytest.raises(tu.Rejected, match="WORKLOAD_DONE"):
        tu.accept(tu.Report.read(TEXT.replace("WORKLOAD_DONE\n", "")))
    with pytest.raises(tu.Rejected, match="golden check: sgemm_naive"):
        tu.accept(tu.Report.read(TEXT.replace("sgemm_naive 256: CORRECT", "sgemm_naive 256: WRONG")))
    with pytest.raises(tu.Rejected, match="n = 1024"):
        tu.accept(tu.Report.read(TEXT.replace("sgemm 1024x1024x1024", "sgemm 1024x1024x1000")))
    with pytest.raises(tu.Rejected, match="membw"):
        tu.accept(tu.Report.read(TEXT.replace("membw read", "membw_read")))
    extra = TEXT.replace("WORKLOAD_DONE", "sgemm_opt 1023x1025x997: WRONG, 0.030 ms/iter, 70000.0 GFLOPS\nWORKLOAD_DONE")
    with pytest.raises(tu.Rejected, match="sgemm_extra:sgemm_opt:1023x1025x997"):
        tu.accept(tu.Report.read(extra))


def test_tegra_text_report_from_the_reference_harness():
    """The reference harness's own text (gpu_workload.c:115-218 formats): no device line, a
    64 MB probe, Tegra numbers -> the Tegra limits accept it."""
    text = ("sgemm 256: CORRECT\nsgemm_naive 256: CORRECT (0 bad cells)\nsgemm 256x256x256: 0.6 ms/iter, 57.6 GFLOPS\n"
            "sgemm 512x512x512: 4.2 ms/iter, 63.6 GFLOPS\nsgemm 1024x1024x1024: 33.2 ms/iter, 64.6 GFLOPS\n"
            "membw read (64MB x40): 0.119 s, 22.3 GB/s\nWORKLOAD_DONE\n")
    r = tu.accept(tu.Report.read(text))
    assert r["arch"] is None and r["membw_mb"] == 64 and r["gbps"] == 22.3


def test_recheck_rejects_unverified_results():
    r = accept_json(report())
    with pytest.raises(tu.Rejected, match="correct = true"):
        tu.recheck({**r, "correct": False})
    with pytest.raises(tu.Rejected, match="n = 1024"):
        tu.recheck({**r, "gflops": {"256": 1.0e3, "512": 2.0e3}})
    with pytest.raises(tu.Rejected, match="no sgemm verdict"):
        tu.recheck({**r, "kernels_verified": []})
    with pytest.raises(tu.Rejected):
        tu.recheck(None)


def fake_harness(tmp_path, script, name="gpu_workload"):
    p = tmp_path / name
    p.write_text("#!/bin/bash\n" + script)
    p.chmod(p.stat().st_mode | stat.S_IXUSR)
    return str(p)


def test_unit_json(tmp_path):
    out = tmp_path / "out.json"
    out.write_text(report() + "\n")
    h = fake_harness(tmp_path, f'[ "$1" = --json ] || exit 9\ncat {out}\n')
    assert tu.Harness(h, "x.co").unit()["gflops"]["1024"] == 79000.0


def test_unit_falls_back_to_text(tmp_path):
    """A harness without --json reads the flag as its code-object path and fails; the unit
    re-runs it without the flag and reads the text lines."""
    out = tmp_path / "out.txt"
    out.write_text(TEXT.split("\n", 1)[1])
    h = fake_harness(tmp_path, f'[ "$1" = --json ] && {{ echo "cannot open --json" >&2; exit 1; }}\ncat {out}\n')
    assert tu.Harness(h, "x.co", arch="gfx950").unit()["gbps"] == 6712.4


def test_unit_failures(tmp_path):
    with pytest.raises(tu.Rejected, match="exited 3: boom"):
        tu.Harness(fake_harness(tmp_path, 'echo "{\\"done\\":false}"; echo boom >&2; exit 3\n'), "x.co").unit()
    with pytest.raises(tu.Rejected, match="exited 4"):
        tu.Harness(fake_harness(tmp_path, 'echo nope >&2; exit 4\n'), "x.co").unit()
    with pytest.raises(tu.Rejected, match="timed out"):
        tu.Harness(fake_harness(tmp_path, "sleep 5\n"), "x.co", timeout=0.5).unit()
    with pytest.raises(tu.Rejected, match="cannot run"):
        tu.Harness(str(tmp_path / "missing"), "x.co").unit()


def test_discover_home(tmp_path):
    """The home lookup order of deploy/cluster/README.md: $CLUSTER_GPU_HOME, ~/switch-l4t-gpu,
    ~/gpu; a home qualifies only with an executable harness and its code object."""
    user, env_home = tmp_path / "user", tmp_path / "env"
    user.mkdir(), env_home.mkdir()
    env = {"CLUSTER_GPU_HOME": str(env_home), "HOME": str(user)}
    assert tu.Harness.discover(env) is None
    fake_harness(env_home, "exit 0\n")
    assert tu.Harness.discover(env) is None                  # no code object yet
    (env_home / "switch_gpu.co").write_bytes(b"\0")
    h = tu.Harness.discover(env, timeout=7)
    assert (h.binary, h.code_object, h.timeout) == (str(env_home / "gpu_workload"), str(env_home / "switch_gpu.co"), 7)
    os.chmod(env_home / "gpu_workload", 0o644)               # not executable: the home does not qualify
    assert tu.Harness.discover(env) is None
    tree = user / "gpu" / "switch-l4t-gpu_amd"               # ~/gpu holding this repo's in-tree build
    (tree / "bin").mkdir(parents=True), (tree / "build").mkdir()
    fake_harness(tree / "bin", "exit 0\n")
    (tree / "build" / "switch_gpu.co").write_bytes(b"\0")
    assert tu.Harness.discover(env).binary == str(tree / "bin" / "gpu_workload")
    first = user / "switch-l4t-gpu"                          # ~/switch-l4t-gpu comes before ~/gpu
    first.mkdir()
    fake_harness(first, "exit 0\n")
    (first / "switch_gpu.co").write_bytes(b"\0")
    assert tu.Harness.discover(env).binary == str(first / "gpu_workload")
    assert tu.Harness.discover({"HOME": str(user)}).binary == str(first / "gpu_workload")


@pytest.mark.gpu
def test_live_harness_report(gpu):
    """The real harness on the GPU: its --json report passes the MI355X limits, and so does its
    text report (the device line names gfx950)."""
    binary = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "gpu_workload")
    co = os.path.join(ROOT, "switch-l4t-gpu_amd", "build", "switch_gpu.co")
    h = tu.Harness(binary, co, timeout=120)
    r = h.unit()
    print("unit result", json.dumps(r), flush=True)
    assert r["correct"] and r["arch"] == "gfx950" and r["membw_mb"] >= tu.MALL_MB
    assert set(r["kernels_verified"]) == {"sgemm", "sgemm_naive", "sgemm_tiled4", "sgemm_opt"}
    tu.recheck(r)
    proc = h._spawn(())                                   # the text form of the same harness
    assert proc.returncode == 0, proc.stderr
    rt = tu.accept(tu.Report.read(proc.stdout))
    assert rt["arch"] == "gfx950" and set(rt["kernels_verified"]) == set(r["kernels_verified"])
