"""Task-queue unit for the gpu_workload harness on MI355X.

A queue worker claims a unit, runs the harness once and hands back a small result dict; the
coordinator re-checks that dict before it trusts it.  Only the contract is shared with the
reference consumer (deploy/cluster/gpu_task_example.py:21-24,57-102; deploy/cluster/README.md):
  * invocation `gpu_workload --json <code object>`; a harness that predates --json reads the
    flag as its code-object path, fails without printing a JSON object, and is then run
    without it and read from its text lines;
  * JSON keys `kernels`, `sgemm` [{n, ms, gflops}], `membw_gbps`, `done`; text lines
    `<kernel> <n>: CORRECT|WRONG`, `sgemm <n>x<n>x<n>: <t> ms/iter, <g> GFLOPS`,
    `membw read ...: <g> GB/s`, and the `WORKLOAD_DONE` sentinel;
  * acceptance: the report is complete, every golden-check verdict is CORRECT (the sgemm one
    present), SGEMM is timed at n = 256, 512 and 1024, and the numbers pass sanity bounds
    that catch garbage, not fraud; one unit may take 50 s;
  * the worker's home lookup: $CLUSTER_GPU_HOME, then ~/switch-l4t-gpu, then ~/gpu.

How this module is organised:
  Report   one normalised record.  The JSON form, the text form and a coordinator's result
           dict are each read into it, so everything after reading has one code path.
  LIMITS   sanity limits per device, picked by the report's `arch` (a gfx950 harness writes
           it; a report without one comes from a Tegra X1 and keeps the reference's limits).
  RULES    the acceptance rules as a table of named checks.  audit() applies all of them and
           returns every finding, so a rejected unit names all of its problems at once.
  Harness  where a harness lives and how it is invoked: a tuple of invocation forms tried
           newest first.
"""
from __future__ import annotations

import json
import os
import re
import subprocess
from dataclasses import dataclass, field

REQUIRED_SIZES = (256, 512, 1024)
UNIT_SECONDS = 50
MALL_MB = 512            # a read-probe buffer at least this large streams HBM, not the 256 MB MALL


class Rejected(ValueError):
    """A harness run or a reported result that must not be accepted; `findings` lists why."""

    def __init__(self, findings):
        self.findings = list(findings)
        super().__init__("; ".join(self.findings))


# ---------------------------------------------------------------------------------------------
# Device limits.  The upper limits sit 5% above the device's peak, so only a number no run can
# produce is refused:
#   tegra-x1  the reference's fixed gates, (1, 1000) for both GFLOPS and GB/s (FMA peak about
#             472 GFLOPS, LPDDR4 25.6 GB/s)
#   gfx950    MI355X: SGEMM on the fp32 matrix cores, 157.3 TFLOP/s dense; the read probe is
#             bounded by HBM3E (8 TB/s) for a buffer past the MALL and by the MALL (about
#             17.2 TB/s) for one that may sit in it.
@dataclass(frozen=True)
class Limits:
    gflops: tuple
    gbps_hbm: tuple
    gbps_mall: tuple

    @classmethod
    def from_peaks(cls, gflops, hbm_gbps, mall_gbps, slack=1.05):
        return cls((1.0, gflops * slack), (1.0, hbm_gbps * slack), (1.0, mall_gbps * slack))


LIMITS = {
    "tegra-x1": Limits((1.0, 1000.0), (1.0, 1000.0), (1.0, 1000.0)),
    "gfx950": Limits.from_peaks(157300.0, 8000.0, 17200.0),
}
UNNAMED_DEVICE = "tegra-x1"


def _number(v):
    return isinstance(v, (int, float)) and not isinstance(v, bool)


def _inside(v, span):
    return _number(v) and span[0] <= v <= span[1]


# ---------------------------------------------------------------------------------------------
# The normalised report.
_END_MARK = {"json": "the done flag is not true", "text": "no WORKLOAD_DONE sentinel",
             "result": "the result does not claim correct = true"}

# Text lines, matched from the start of each line (indented diagnostics never match).
_LINE_KINDS = (
    ("verdict", re.compile(r"(?P<kernel>sgemm\w*) (?P<n>\d+): (?P<verdict>CORRECT|WRONG)\b")),
    ("extra", re.compile(r"(?P<kernel>sgemm\w*) (?P<m>\d+)x(?P<n>\d+)x(?P<k>\d+): (?P<verdict>CORRECT|WRONG),")),
    ("timing", re.compile(r"sgemm (?P<m>\d+)x(?P<n>\d+)x(?P<k>\d+): [\d.]+ ms/iter, (?P<gflops>[\d.]+) GFLOPS")),
    ("membw", re.compile(r"membw read\b(?: \((?P<mb>\d+)MB)?.*?(?P<gbps>[\d.]+) GB/s")),
    ("device", re.compile(r"device: .*\((?P<arch>[\w-]+)\)\s*$")),
    ("end", re.compile(r"WORKLOAD_DONE\b")),
)


def _extra_name(kernel, m, n, k):
    return f"sgemm_extra:{kernel}:{m}x{n}x{k}"


@dataclass
class Report:
    form: str                                       # "json", "text" or "result"
    end_mark: bool = False                          # done: true / WORKLOAD_DONE / correct: true
    verdicts: dict = field(default_factory=dict)    # golden-check name -> verdict string
    gflops: dict = field(default_factory=dict)      # square size n -> GFLOPS of the sgemm kernel
    gbps: object = None                             # the read probe's GB/s, as reported
    membw_mb: int | None = None                     # the read probe's buffer size, when stated
    arch: str | None = None

    @classmethod
    def read(cls, stdout: str, arch: str | None = None) -> "Report":
        """Harness stdout in either form; `arch` names the device when the text does not."""
        if stdout.lstrip().startswith("{"):
            return cls.from_json(stdout)
        rep = cls.from_text(stdout)
        rep.arch = rep.arch or arch
        return rep

    @classmethod
    def from_json(cls, text: str) -> "Report":
        try:
            data = json.loads(text)
        except json.JSONDecodeError as exc:
            raise Rejected([f"JSON report unreadable (truncated?): {exc}"]) from exc
        if not isinstance(data, dict):
            raise Rejected(["JSON report incomplete: not an object"])
        rep = cls("json", end_mark=data.get("done") is True, gbps=data.get("membw_gbps"),
                  arch=data.get("arch") or None)
        mb = data.get("membw_mb")
        rep.membw_mb = mb if _number(mb) else None
        kernels = data.get("kernels")
        if isinstance(kernels, dict):
            rep.verdicts.update(kernels)
        for row in data.get("sgemm_extra") or ():
            row = row if isinstance(row, dict) else {}
            rep.verdicts[_extra_name(row.get("kernel"), row.get("m"), row.get("n"), row.get("k"))] = row.get("verdict")
        for row in data.get("sgemm") or ():
            if isinstance(row, dict) and isinstance(row.get("n"), int) and _number(row.get("gflops")):
                rep.gflops[row["n"]] = float(row["gflops"])
        return rep

    @classmethod
    def from_text(cls, text: str) -> "Report":
        rep = cls("text")
        for line in text.splitlines():
            for kind, pat in _LINE_KINDS:
                m = pat.match(line)
                if m is None:
                    continue
                g = m.groupdict()
                if kind == "verdict":
                    rep.verdicts[g["kernel"]] = g["verdict"]
                elif kind == "extra":
                    rep.verdicts[_extra_name(g["kernel"], g["m"], g["n"], g["k"])] = g["verdict"]
                elif kind == "timing" and g["m"] == g["n"] == g["k"]:
                    rep.gflops[int(g["n"])] = float(g["gflops"])
                elif kind == "membw" and rep.gbps is None:
                    rep.gbps = float(g["gbps"])
                    rep.membw_mb = int(g["mb"]) if g["mb"] else None
                elif kind == "device":
                    rep.arch = g["arch"].split(":")[0]
                elif kind == "end":
                    rep.end_mark = True
                break
        return rep

    @classmethod
    def from_result(cls, result) -> "Report":
        """A result dict as summary() makes it, e.g. after a JSON round trip to the coordinator."""
        d = result if isinstance(result, dict) else {}
        rep = cls("result", end_mark=d.get("correct") is True, gbps=d.get("gbps"),
                  membw_mb=d.get("membw_mb"), arch=d.get("arch"))
        rep.verdicts = {k: "CORRECT" for k in d.get("kernels_verified") or ()}
        for k, v in (d.get("gflops") or {}).items():
            if str(k).isdigit():
                rep.gflops[int(k)] = v
        return rep

    def summary(self) -> dict:
        """The result dict a worker reports: JSON-ready, string size keys."""
        return {"correct": True, "kernels_verified": sorted(k for k in self.verdicts if ":" not in k),
                "arch": self.arch, "membw_mb": self.membw_mb,
                "gflops": {str(n): round(float(self.gflops[n]), 1) for n in sorted(self.gflops)},
                "gbps": round(float(self.gbps), 1)}


# ---------------------------------------------------------------------------------------------
# Acceptance rules.  Each takes the report and its device's limits (None when the device has
# none) and yields findings.
def _rule_device(rep, lim):
    if lim is None:
        yield f"no sanity bounds for device {rep.arch!r}"


def _rule_complete(rep, lim):
    if not rep.end_mark:
        yield f"report incomplete: {_END_MARK[rep.form]}"


def _rule_golden(rep, lim):
    if "sgemm" not in rep.verdicts:
        yield "no sgemm verdict: the harness's golden check did not run"
    wrong = sorted(str(k) for k, v in rep.verdicts.items() if v != "CORRECT")
    if wrong:
        yield f"failed the harness's CPU golden check: {', '.join(wrong)}"


def _rule_timed(rep, lim):
    for n in REQUIRED_SIZES:
        v = rep.gflops.get(n)
        if v is None:
            yield f"no SGEMM timing at n = {n}"
        elif lim is not None and not _inside(v, lim.gflops):
            yield f"SGEMM n = {n}: {v!r} GFLOPS outside the sanity bounds {lim.gflops}"


def _rule_membw(rep, lim):
    if lim is None:
        return
    span = lim.gbps_hbm if rep.membw_mb is None or rep.membw_mb >= MALL_MB else lim.gbps_mall
    if not _inside(rep.gbps, span):
        yield f"membw {rep.gbps!r} GB/s missing or outside the sanity bounds {span}"


RULES = (("device", _rule_device), ("complete", _rule_complete), ("golden", _rule_golden),
         ("timed", _rule_timed), ("membw", _rule_membw))


def limits_for(arch: str | None) -> Limits | None:
    return LIMITS.get((arch or UNNAMED_DEVICE).split(":")[0])


def audit(rep: Report) -> list:
    """Every finding against the report (empty: acceptable)."""
    lim = limits_for(rep.arch)
    return [f for _, rule in RULES for f in rule(rep, lim)]


def accept(rep: Report) -> dict:
    """The report's result dict, or Rejected naming every finding."""
    findings = audit(rep)
    if findings:
        raise Rejected(findings)
    return rep.summary()


def recheck(result) -> None:
    """Coordinator side: re-apply the same rules to a worker's reported result dict."""
    findings = audit(Report.from_result(result))
    if findings:
        raise Rejected(findings)


# ---------------------------------------------------------------------------------------------
# The harness.
_LAYOUTS = ((("switch-l4t-gpu_amd", "bin", "gpu_workload"), ("switch-l4t-gpu_amd", "build", "switch_gpu.co")),
            (("gpu_workload",), ("switch_gpu.co",)))


@dataclass
class Harness:
    binary: str
    code_object: str
    timeout: float = UNIT_SECONDS
    arch: str | None = None          # the device, for a text report that does not name one
    extra_args: tuple = ()

    # (form, flags placed before the code object), newest first
    FORMS = (("json", ("--json",)), ("text", ()))

    @classmethod
    def discover(cls, environ=None, **kw) -> "Harness | None":
        """The first home holding an executable harness and its code object, in the lookup
        order $CLUSTER_GPU_HOME, ~/switch-l4t-gpu, ~/gpu; None when this machine has none."""
        env = os.environ if environ is None else environ
        homes = [env["CLUSTER_GPU_HOME"]] if env.get("CLUSTER_GPU_HOME") else []
        user = env.get("HOME") or os.path.expanduser("~")
        homes += [os.path.join(user, d) for d in ("switch-l4t-gpu", "gpu")]
        for home in homes:
            for bin_parts, co_parts in _LAYOUTS:
                binary, co = os.path.join(home, *bin_parts), os.path.join(home, *co_parts)
                if os.path.isfile(binary) and os.access(binary, os.X_OK) and os.path.isfile(co):
                    return cls(binary, co, **kw)
        return None

    def _spawn(self, flags):
        argv = [self.binary, *flags, *self.extra_args, self.code_object]
        try:
            return subprocess.run(argv, capture_output=True, text=True, timeout=self.timeout)
        except subprocess.TimeoutExpired as exc:
            raise Rejected([f"harness timed out after {self.timeout} s"]) from exc
        except OSError as exc:
            raise Rejected([f"cannot run the harness {self.binary!r}: {exc}"]) from exc

    def report(self) -> Report:
        """Run the harness in the newest form it understands and read its report."""
        for i, (form, flags) in enumerate(self.FORMS):
            proc = self._spawn(flags)
            if proc.returncode == 0:
                return Report.read(proc.stdout, self.arch)
            # A JSON-capable harness that failed still starts its stdout with an object; an
            # older one took the flag for its code-object path, so the next form is tried.
            understood = form != "json" or proc.stdout.lstrip().startswith("{")
            if understood or i + 1 == len(self.FORMS):
                raise Rejected([f"harness exited {proc.returncode}: {proc.stderr.strip()[:300]}"])
        raise AssertionError("unreachable")

    def unit(self) -> dict:
        """One task unit: the checked result dict, or Rejected."""
        return accept(self.report())


if __name__ == "__main__":
    import sys

    h = Harness.discover()
    if h is None:
        sys.exit("no GPU home ($CLUSTER_GPU_HOME, ~/switch-l4t-gpu, ~/gpu) holds a built harness")
    try:
        print(json.dumps(h.unit(), indent=2))
    except Rejected as exc:
        sys.exit(f"unit rejected: {exc}")
