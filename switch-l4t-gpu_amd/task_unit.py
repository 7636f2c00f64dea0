"""Task-queue unit around the gpu_workload harness: run it, check its report, re-check a
reported result -- the consumer contract of deploy/cluster/gpu_task_example.py:21-128, with
sanity bounds sized per device instead of the Tegra X1's fixed (1, 1000).

A unit runs `gpu_workload --json <code_object>` (a harness built before --json is re-run
without it and its text lines are read), and accepts the run only if
  - the report is complete: the JSON `done` flag is true (text: the WORKLOAD_DONE sentinel);
  - every kernel verdict of the harness's on-device CPU golden check is CORRECT (the sgemm
    verdict must be present), and so is every added `sgemm_extra` verdict;
  - SGEMM timings exist for 256, 512 and 1024, and they and the read bandwidth lie inside the
    device's sanity bounds (BOUNDS) -- garbage gates, not a second correctness check.
The device comes from the report's `arch` key (gpu_workload --json on gfx950 adds it); a
report without one is a Tegra X1 report and gets the reference's bounds.  verify_unit()
re-checks a reported result dict on the coordinator side with the same bounds.
"""
from __future__ import annotations

import json
import re
import subprocess

SIZES = (256, 512, 1024)
TIMEOUT_S = 50

# Sanity bounds (lower, upper) per device.  Upper bounds sit 5% above the device's peak, so
# only numbers no run can produce are rejected:
#   tegra-x1  the reference's gates (gpu_task_example.py:23-24; FMA peak ~472 GFLOPS, LPDDR4
#             25.6 GB/s)
#   gfx950    MI355X: SGEMM runs on the fp32 matrix cores, 157.3 TFLOP/s dense peak -> 165,165
#             GFLOPS; the read probe is bounded by HBM3E (8 TB/s -> 8,400 GB/s) when its buffer
#             is larger than the 256 MB MALL (membw_mb >= 512; the harness default is 1024),
#             and by the MALL's peak (about 17.2 TB/s -> 18,060 GB/s) when it may sit in it.
BOUNDS = {
    "tegra-x1": {"gflops": (1.0, 1000.0), "gbps": (1.0, 1000.0), "gbps_mall": (1.0, 1000.0)},
    "gfx950": {"gflops": (1.0, 157300.0 * 1.05), "gbps": (1.0, 8000.0 * 1.05), "gbps_mall": (1.0, 17200.0 * 1.05)},
}
MALL_MB = 512            # a probe buffer at least this large streams HBM, not the 256 MB MALL

_VERDICT_LINE = re.compile(r"^(sgemm(?:_\w+)?) (\d+): (CORRECT|WRONG)\b", re.M)
_PERF_LINE = re.compile(r"^sgemm (\d+)x\1x\1: [\d.]+ ms/iter, ([\d.]+) GFLOPS", re.M)
_MEMBW_LINE = re.compile(r"^membw read \((\d+)MB[^)]*\).* ([\d.]+) GB/s|^membw read .* ([\d.]+) GB/s", re.M)


class UnitError(ValueError):
    """The unit's report is incomplete, wrong, or outside the device's sanity bounds."""


def bounds_for(arch: str | None) -> dict:
    if not arch:
        return BOUNDS["tegra-x1"]
    key = arch.split(":")[0]
    if key not in BOUNDS:
        raise UnitError(f"no sanity bounds for device {arch!r}")
    return BOUNDS[key]


def check_numbers(gflops: dict, gbps, arch: str | None = None, membw_mb: int | None = None) -> None:
    """Every required SGEMM size present with GFLOPS inside the device's bounds, and the read
    bandwidth inside the HBM bounds (or the MALL bounds for a buffer that may sit in the MALL)."""
    b = bounds_for(arch)
    lo, hi = b["gflops"]
    for size in map(str, SIZES):
        v = gflops.get(size)
        if not isinstance(v, (int, float)) or isinstance(v, bool) or not lo <= v <= hi:
            raise UnitError(f"gflops[{size}] = {v!r} missing or outside the sanity bounds ({lo}, {hi})")
    glo, ghi = b["gbps"] if (membw_mb is None or membw_mb >= MALL_MB) else b["gbps_mall"]
    if not isinstance(gbps, (int, float)) or isinstance(gbps, bool) or not glo <= gbps <= ghi:
        raise UnitError(f"membw {gbps!r} GB/s missing or outside the sanity bounds ({glo}, {ghi})")


def parse_json(out: str) -> dict:
    """A `gpu_workload --json` report -> result dict (UnitError on any problem)."""
    try:
        data = json.loads(out)
    except json.JSONDecodeError as exc:
        raise UnitError(f"harness JSON unreadable (truncated?): {exc}") from exc
    if not isinstance(data, dict) or data.get("done") is not True:
        raise UnitError("harness JSON incomplete: the done flag is not true")
    kernels = data.get("kernels")
    if not isinstance(kernels, dict) or "sgemm" not in kernels:
        raise UnitError("harness JSON has no sgemm verdict")
    failed = sorted(k for k, v in kernels.items() if v != "CORRECT")
    failed += sorted(f"sgemm_extra:{r.get('kernel')}:{r.get('m')}x{r.get('n')}x{r.get('k')}"
                     for r in data.get("sgemm_extra") or [] if not isinstance(r, dict) or r.get("verdict") != "CORRECT")
    if failed:
        raise UnitError(f"kernels failed the harness's CPU golden check: {failed}")
    gflops = {}
    for row in data.get("sgemm") or []:
        if isinstance(row, dict) and isinstance(row.get("n"), int) and isinstance(row.get("gflops"), (int, float)):
            gflops[str(row["n"])] = float(row["gflops"])
    missing = [s for s in map(str, SIZES) if s not in gflops]
    if missing:
        raise UnitError(f"no SGEMM timing for size(s) {missing}")
    arch, mb = data.get("arch"), data.get("membw_mb")
    check_numbers(gflops, data.get("membw_gbps"), arch, mb)
    return {"correct": True, "kernels_verified": sorted(kernels), "arch": arch, "membw_mb": mb,
            "gflops": {k: round(v, 1) for k, v in gflops.items()}, "gbps": round(float(data["membw_gbps"]), 1)}


def parse_text(out: str, arch: str | None = None) -> dict:
    """The harness's human-readable lines (a harness without --json) -> result dict."""
    if "WORKLOAD_DONE" not in out:
        raise UnitError("harness output incomplete: no WORKLOAD_DONE sentinel")
    verdicts = {m.group(1): m.group(3) for m in _VERDICT_LINE.finditer(out)}
    if "sgemm" not in verdicts:
        raise UnitError("harness printed no sgemm verdict")
    failed = sorted(k for k, v in verdicts.items() if v != "CORRECT")
    if failed:
        raise UnitError(f"kernels failed the harness's CPU golden check: {failed}")
    gflops = {m.group(1): float(m.group(2)) for m in _PERF_LINE.finditer(out)}
    missing = [s for s in map(str, SIZES) if s not in gflops]
    if missing:
        raise UnitError(f"no SGEMM timing for size(s) {missing}")
    m = _MEMBW_LINE.search(out)
    if m is None:
        raise UnitError("harness printed no membw line")
    mb = int(m.group(1)) if m.group(1) else None
    gbps = float(m.group(2) or m.group(3))
    check_numbers(gflops, gbps, arch, mb)
    return {"correct": True, "kernels_verified": sorted(verdicts), "arch": arch, "membw_mb": mb,
            "gflops": {k: round(v, 1) for k, v in gflops.items()}, "gbps": round(gbps, 1)}


def run_unit(binary: str, code_object: str, timeout: float = TIMEOUT_S, arch: str | None = None,
             extra_args: tuple = ()) -> dict:
    """One task unit: run the harness on a code object and return its checked result.
    `arch` names the device for a harness whose text report does not (JSON reports carry it)."""
    def run(args):
        try:
            return subprocess.run([binary, *args], capture_output=True, text=True, timeout=timeout)
        except subprocess.TimeoutExpired as exc:
            raise UnitError(f"harness timed out after {timeout} s") from exc
        except OSError as exc:
            raise UnitError(f"cannot run the harness {binary!r}: {exc}") from exc

    proc = run(["--json", *extra_args, code_object])
    if proc.returncode != 0 and not proc.stdout.lstrip().startswith("{"):
        proc = run([*extra_args, code_object])        # a harness that reads --json as a path
    if proc.returncode != 0:
        raise UnitError(f"harness exited {proc.returncode}: {proc.stderr.strip()[:300]}")
    out = proc.stdout
    return parse_json(out) if out.lstrip().startswith("{") else parse_text(out, arch)


def verify_unit(result: dict) -> None:
    """Coordinator-side re-check of a reported result dict."""
    if not isinstance(result, dict) or result.get("correct") is not True:
        raise UnitError("result does not report correct = true (no golden check)")
    check_numbers(result.get("gflops") or {}, result.get("gbps"), result.get("arch"), result.get("membw_mb"))
