"""The instruction sequence the cross-block hand-off relies on, read from the gfx950 code objects
this repository builds (CPU only: the AMD disassembly of our own kernels).

The hand-off (split-K SGEMM, the split batched GEMM, the Qwen prefill GEMM, the decode
attention's position chunks) has no release on the writer's side.  What takes its place is
this sequence, and this test fails if the compiler stops emitting it:

  writer  global_store_dword ... sc1      partial records written through past the per-XCD L2
          s_waitcnt vmcnt(0)              every one of the wave's stores acknowledged
          s_barrier                       every wave of the block past that point
          global_atomic_add ... sc0       then the counter add (returns the old count)
  reader  buffer_inv sc1                  the last arriver's agent-scope acquire
          global_load_dword ... sc1       the partial records read coherently

The order is checked along the kernel's text.  For the writer, the last sc1 store before the
first counter add must be followed, before that add, by vmcnt(0) and a barrier.  For the
reader, an acquire must follow the add and come before the first sc1 load after it."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "switch-l4t-gpu_amd", "build")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"

KERNELS = [
    ("switch_gpu", "sgemm_splitk"),              # split-K SGEMM (also the allocation-free entry)
    ("gpt2_kernels", "gemv_multi_splitk"),       # the split batched GEMM
    ("sgpu_decode", "sgpu_pf_gemm"),             # the Qwen prefill's split GEMM
    ("sgpu_decode", "sgpu_dec_attn32"),          # decode attention, chunked caches
    ("sgpu_decode", "sgpu_dec_attn64"),
    ("sgpu_decode", "sgpu_dec_attn128"),
]


def kernel_text(co, sym):
    out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", os.path.join(BUILD, co + ".co")],
                         capture_output=True, text=True, check=True).stdout
    lines, on = [], False
    for line in out.splitlines():
        if re.match(r"^[0-9a-f]+ <.*>:", line):
            on = line.rstrip().endswith(f"<{sym}>:")
            continue
        if on:
            ins = line.split("//")[0].strip()
            if ins:
                lines.append(ins)
    return lines


def sequence_error(text):
    """None when the instruction list holds the hand-off sequence, else what is wrong."""
    adds = [k for k, i in enumerate(text) if i.startswith("global_atomic_add")]
    if not adds:
        return "no counter add"
    add = adds[0]
    stores = [k for k in range(add) if text[k].startswith("global_store_dword") and text[k].split()[-1] == "sc1"]
    if not stores:
        return "no write-through (sc1) store before the counter add"
    between = text[stores[-1] + 1:add]
    wait = next((k for k, i in enumerate(between) if re.match(r"s_waitcnt\b.*vmcnt\(0\)", i)), None)
    if wait is None:
        return "the stores are not waited for before the counter add"
    if not any(i == "s_barrier" for i in between[wait + 1:]):
        return "no barrier between the wait and the add"
    after = text[add + 1:]
    inv = next((k for k, i in enumerate(after) if i == "buffer_inv sc1"), None)
    if inv is None:
        return "no agent-scope acquire after the counter add"
    first_load = next((k for k, i in enumerate(after) if i.startswith("global_load_dword") and i.split()[-1] == "sc1"),
                      None)
    if first_load is None or first_load < inv:
        return "partials are not read with sc1 loads after the acquire"
    # no release was put back on the writer's side (it measured +55% on split SGEMM)
    if any(i.startswith("buffer_wbl2") for i in text[:add]):
        return "an L2 write-back appeared before the add"
    return None


GOOD = ["global_store_dword v1, v2, s[0:1] sc1", "s_waitcnt vmcnt(0) lgkmcnt(0)", "s_barrier",
        "global_atomic_add v0, v1, v2, s[2:3] sc0", "s_cbranch_vccz 5", "buffer_inv sc1", "s_barrier",
        "global_load_dword v3, v1, s[0:1] sc1"]


@pytest.mark.parametrize("mistake,edit", [
    ("plain store", lambda t: [t[0].replace(" sc1", "")] + t[1:]),
    ("no wait", lambda t: [t[0]] + t[2:]),
    ("barrier before the wait", lambda t: [t[0], t[2], t[1]] + t[3:]),
    ("no acquire", lambda t: t[:5] + t[6:]),
    ("plain partial loads", lambda t: t[:-1] + [t[-1].replace(" sc1", "")]),
    ("write-back put back", lambda t: ["buffer_wbl2 sc1"] + t),
])
def test_sequence_check_catches(mistake, edit):
    """The check itself: the sequence above passes, and each single mistake is caught."""
    assert sequence_error(GOOD) is None
    assert sequence_error(edit(list(GOOD))) is not None, mistake


@pytest.mark.skipif(not os.path.exists(OBJDUMP), reason="llvm-objdump not installed")
@pytest.mark.parametrize("co,sym", KERNELS)
def test_handoff_sequence(co, sym):
    if not os.path.exists(os.path.join(BUILD, co + ".co")):
        pytest.skip("code objects not built")
    text = kernel_text(co, sym)
    assert text, f"{sym} not found in {co}.co"
    err = sequence_error(text)
    assert err is None, err
