"""No kernel reads its argument segment with vector loads (CPU only: the AMD disassembly of the
gfx950 code objects this repository builds).

At wave launch s[0:1] holds the address of the kernel-argument segment.  The first 14 dwords
of it arrive preloaded in SGPRs, and later dwords are read with scalar loads.  HIP's blockDim
can instead compile to 16-bit vector loads of the hidden group-size / remainder fields
(global_load_ushort from s[0:1] + 40 + 12 or 18).  Those loads run one after another, through
the vector cache that a streaming kernel keeps full, before the block's first useful load.
On the by-name lm_head GEMV (18992 blocks) they cost 3.7 us per launch.

The check follows the SGPRs derived from s[0:1] by scalar arithmetic (a scalar load's result
is a value, not an address, so it ends the derivation) and fails on any vector memory
instruction whose SGPR address comes from them."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "switch-l4t-gpu_amd", "build")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
CODE_OBJECTS = ["switch_gpu", "gemv", "gpt2_kernels", "qwen_kernels", "sgpu_tuned", "sgpu_decode", "sgpu_probe"]

_SREG = re.compile(r"\bs(\d+)\b|\bs\[(\d+):(\d+)\]")


def sregs(operand):
    """The scalar registers an operand string names."""
    out = set()
    for m in _SREG.finditer(operand):
        if m.group(1) is not None:
            out.add(int(m.group(1)))
        else:
            out.update(range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def kernels(co):
    """{kernel name: [instruction, ...]} of one code object."""
    out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", os.path.join(BUILD, co + ".co")],
                         capture_output=True, text=True, check=True).stdout
    ks, cur = {}, None
    for line in out.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.*)>:", line)
        if m:
            cur = ks.setdefault(m.group(1), [])
            continue
        if cur is not None:
            ins = line.split("//")[0].strip()
            if ins and not ins.startswith("s_nop"):
                cur.append(ins)
    return ks


# the scalar operations that carry an address forward (an offset added, a copy, a choice)
_ADDRESS_OPS = ("s_add_u32", "s_addc_u32", "s_add_i32", "s_mov_b32", "s_mov_b64", "s_cselect_b32", "s_cselect_b64")


def argument_vector_loads(text):
    """The vector memory instructions whose SGPR address derives from s[0:1]."""
    derived, bad = {0, 1}, []
    for ins in text:
        op, _, rest = ins.partition(" ")
        ops = [o.strip() for o in rest.split(",")] if rest else []
        if op.startswith(("global_", "buffer_", "flat_")):
            if any(sregs(o) & derived for o in ops[1:]):
                bad.append(ins)
            continue
        if not ops:
            continue
        dst = sregs(ops[0])                           # SGPRs written (also by v_readlane and the like)
        if not dst or op.startswith(("s_cmp", "s_bitcmp", "s_cbranch", "s_branch", "s_waitcnt", "s_barrier")):
            continue
        if op.startswith(_ADDRESS_OPS) and any(sregs(o) & derived for o in ops[1:]):
            derived |= dst
        else:
            derived -= dst                            # a loaded or computed value, not an address
    return bad


# the prologue HIP's blockDim produced in the by-name GEMV symbols, and the form that replaced it
OLD = ["s_add_u32 s0, s0, 40", "s_addc_u32 s1, s1, 0", "s_cmp_lt_u32 s16, s12", "s_cselect_b32 s2, 12, 18",
       "s_add_u32 s2, s0, s2", "s_addc_u32 s3, s1, 0", "v_mov_b32_e32 v0, 0", "global_load_ushort v1, v0, s[2:3]"]
NEW = ["s_lshr_b32 s19, s15, 16", "s_add_u32 s0, s0, 40", "s_addc_u32 s1, s1, 0", "s_and_b32 s15, s15, 0xffff",
       "s_cmpk_lg_i32 s15, 0x100", "s_load_dword s2, s[0:1], 0x10", "s_waitcnt lgkmcnt(0)",
       "s_load_dwordx4 s[4:7], s[2:3], 0x0", "global_load_dwordx4 v[8:11], v2, s[2:3]",
       "global_load_dwordx4 v[8:11], v2, s[46:47]"]


def test_check_catches_the_old_prologue():
    assert argument_vector_loads(OLD) == ["global_load_ushort v1, v0, s[2:3]"]
    assert argument_vector_loads(NEW) == []
    # the derivation survives a 64-bit move and ends at a scalar load into the same registers or
    # at arithmetic that makes a value of the register
    assert argument_vector_loads(["s_mov_b64 s[8:9], s[0:1]", "global_load_dword v1, v0, s[8:9]"])
    assert not argument_vector_loads(["s_load_dwordx2 s[0:1], s[0:1], 0x0", "global_load_dword v1, v0, s[0:1]"])
    assert not argument_vector_loads(["s_mul_i32 s1, s1, s4", "s_mov_b32 s0, s6",
                                      "global_atomic_add v1, v2, v1, s[0:1] sc0"])
    assert not argument_vector_loads(["s_add_u32 s18, s0, 64", "s_addc_u32 s19, s1, 0", "v_readlane_b32 s18, v124, 0",
                                      "v_readlane_b32 s19, v124, 1", "global_atomic_add v1, v2, v1, s[18:19] sc0"])
    # the merged y and z group sizes (bytes 14..17, not dword-aligned) read by a vector load
    assert argument_vector_loads(["s_add_u32 s0, s0, 40", "s_addc_u32 s1, s1, 0",
                                  "global_load_dword v0, v0, s[0:1] offset:14"])


@pytest.mark.skipif(not os.path.exists(OBJDUMP), reason="llvm-objdump not installed")
@pytest.mark.parametrize("co", CODE_OBJECTS)
def test_no_vector_loads_of_kernel_arguments(co):
    if not os.path.exists(os.path.join(BUILD, co + ".co")):
        pytest.skip("code objects not built")
    ks = kernels(co)
    assert ks, f"no kernels in {co}.co"
    bad = {k: v for k, v in ((k, argument_vector_loads(t)) for k, t in ks.items()) if v}
    assert not bad, bad
