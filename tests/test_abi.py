"""The drop-in boundary, checked without a GPU: libswitchgpu.so loads, exports every function
include/switch_gpu.h declares, embeds the gfx950 code objects with the reference kernel
names, and rejects bad arguments before touching a device.  CPU only."""
import ctypes as ct
import struct

import numpy as np
import pytest

# Kernel names each reference module exports (switch_gpu.cu, gemv.cu, gpt2_kernels.cu,
# qwen_kernels.cu) and that hosts resolve by name (gpu_workload.c:69-74, gemv_test.c:68-72,
# gpt2_engine.c:119-128, qwen_engine.c:148-155); a missing one is fatal to those hosts.
REFERENCE_KERNELS = {
    "switch_gpu": {"sgemm_tiled", "sgemm_tiled4", "sgemm_opt", "sgemm_naive", "membw_read4",
                   "sgemm_opt256", "sgemm_splitk", "sgemm_small16",
                   "sgemm_small32", "sgemm_kwave", "sgemm_kwave_edge", "sgemm_kwave_wide",
                   "sgemm_kwave_edge_wide", "sgemm_kwave128"},   # the last nine are added members
                                                      # (no reference counterpart)
    "gemv": {"gemv", "gemv4", "gemv_warp"},
    "gpt2_kernels": {"gemv_warp", "gemv_warp_b", "gemv_multi", "layernorm", "gelu", "add_bias", "add2",
                     "attn_scores", "attn_softmax", "attn_mix"},
    "qwen_kernels": {"gemv_h", "rmsnorm", "rope", "swiglu", "attn_scores_gqa", "attn_softmax",
                     "attn_mix_gqa", "add2"},
}


def elf_kernels(blob: bytes):
    """Names of the kernel descriptors (<name>.kd) in an AMDGPU ELF code object, and e_flags."""
    assert blob[:4] == b"\x7fELF" and blob[4] == 2, "64-bit ELF"
    e_machine, = struct.unpack_from("<H", blob, 18)
    e_flags, = struct.unpack_from("<I", blob, 48)
    e_shoff, = struct.unpack_from("<Q", blob, 40)
    e_shentsize, e_shnum = struct.unpack_from("<HH", blob, 58)
    secs = [struct.unpack_from("<IIQQQQIIQQ", blob, e_shoff + i * e_shentsize) for i in range(e_shnum)]
    names = set()
    for s in secs:
        if s[1] in (2, 11):                     # SHT_SYMTAB / SHT_DYNSYM
            strtab = secs[s[6]]
            for j in range(s[5] // 24):
                st_name, = struct.unpack_from("<I", blob, s[4] + j * 24)
                end = blob.index(b"\0", strtab[4] + st_name)
                nm = blob[strtab[4] + st_name:end].decode()
                if nm.endswith(".kd"):
                    names.add(nm[:-3])
    return e_machine, e_flags, names


def test_library_exports_every_header_function(sg):
    L = sg.lib()
    declared = sg.header_functions()
    assert len(declared) >= 40
    missing = [n for n in declared if not hasattr(L, n)]
    assert not missing, missing
    # and the binding covers them all
    assert set(declared) <= set(sg._SIGS), set(declared) - set(sg._SIGS)


@pytest.mark.parametrize("module", sorted(REFERENCE_KERNELS) + ["sgpu_tuned", "sgpu_probe"])
def test_code_objects_embedded(sg, module):
    size = ct.c_size_t()
    p = sg.lib().sgpu_code_object(module.encode(), ct.byref(size))
    assert p and size.value > 1000
    blob = ct.string_at(p, size.value)
    machine, flags, names = elf_kernels(blob)
    assert machine == 224                        # EM_AMDGPU
    assert flags & 0xFF == 0x4F                  # EF_AMDGPU_MACH_AMDGCN_GFX950
    assert flags & 0x300 != 0x300                # not an xnack+ code object
    if module in REFERENCE_KERNELS:
        assert REFERENCE_KERNELS[module] <= names, REFERENCE_KERNELS[module] - names
    elif module == "sgpu_probe":
        assert {"sgpu_probe_stream", "sgpu_probe_link", "sgpu_probe_mfma"} <= names
    else:
        assert {f"sgpu_gemv_h_l16_s7", "sgpu_gemv_f32_l64_s3", "sgpu_embed_h"} <= names


def test_unknown_code_object(sg):
    assert sg.lib().sgpu_code_object(b"nope", None) is None


def test_geometry_contract(sg):
    g, b = (ct.c_uint * 3)(), (ct.c_uint * 3)()
    L = sg.lib()
    assert L.sgpu_kernel_geometry(b"sgemm_opt", 4096, 4096, 4096, g, b) == 0
    assert tuple(b) == (256, 1, 1) and g[0] == 32 * 16          # one 128x256 tile per block
    assert L.sgpu_kernel_geometry(b"sgemm_opt256", 4096, 4096, 4096, g, b) == 0
    assert tuple(b) == (256, 1, 1) and g[0] == 16 * 16          # one 256x256 tile per block
    assert L.sgpu_kernel_geometry(b"sgemm_tiled4", 4096, 4096, 4096, g, b) == 0
    assert tuple(b) == (256, 1, 1) and g[0] == 32 * 32          # one 128x128 tile per block
    assert L.sgpu_kernel_geometry(b"sgemm_kwave128", 4096, 4096, 4096, g, b) == 0
    assert tuple(b) == (256, 1, 1) and g[0] == 32 * 32          # one 128x128 tile per block
    assert L.sgpu_kernel_geometry(b"sgemm_kwave", 1024, 1024, 1024, g, b) == 0
    assert tuple(b) == (256, 1, 1) and g[0] == 16 * 16          # one 64x64 tile per block
    assert L.sgpu_kernel_geometry(b"sgemm_tiled", 1023, 1025, 997, g, b) == 0
    assert g[0] == 16 * 17                                       # ceil(1023/64) * ceil(1025/64)
    assert L.sgpu_kernel_geometry(b"sgemm_naive", 100, 50, 7, g, b) == 0
    assert tuple(b) == (16, 16, 1) and g[0] == 4 and g[1] == 7
    assert L.sgpu_kernel_geometry(b"gemv_h", 0, 151936, 896, g, b) == 0
    assert b[0] == 256 and g[0] >= 1
    assert L.sgpu_kernel_geometry(b"no_such_kernel", 1, 1, 1, g, b) == sg.SGPU_ERR_NO_KERNEL
    assert L.sgpu_kernel_geometry(b"sgemm_opt", -1, 1, 1, g, b) == sg.SGPU_ERR_INVALID_ARG


def test_argument_errors_before_device(sg):
    """Shape errors are reported as SGPU_ERR_INVALID_ARG without any device work, and empty
    problems are no-ops (the CPU container has no device, so anything else would fail)."""
    L = sg.lib()
    assert L.sgpu_sgemm_opt(None, None, None, -1, 4, 4, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_opt(None, None, None, 0, 4, 4, None) == 0
    assert L.sgpu_sgemm_tiled(None, None, None, 4, 4, 4, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_gemv_h(None, None, None, None, 896, 0, None) == 0
    assert L.sgpu_gemv_h(None, None, None, None, -1, 5, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_gemv_multi(None, None, None, None, 8, 8, -2, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_rope(None, None, None, 1, 2, 7, 0, None) == sg.SGPU_ERR_INVALID_ARG  # odd HD
    assert L.sgpu_attn_scores_gqa(None, None, None, 1, 0.1, 3, 128, 64, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_membw_read4(None, None, 16, 1, None, None) == sg.SGPU_ERR_INVALID_ARG
    # engine entry points: NULL engines and out-of-range paths are rejected
    assert L.sgpu_qwen_set_path(None, 1) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_gpt2_set_path(None, 1) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_qwen_generate(None, None, 1, 1, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_gpt2_generate(None, None, 1, 1, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_gpt2_forward(None, 0, 0, 1, None, 0) == sg.SGPU_ERR_INVALID_ARG
    # split-K: bad split counts and problems past the workspace are rejected up front
    assert L.sgpu_sgemm_splitk(None, None, None, 64, 64, 64, 0, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_splitk(None, None, None, 4096, 4096, 4096, 2, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_splitk(None, None, None, 0, 64, 64, 2, None) == 0
    assert L.sgpu_sgemm_small(None, None, None, 64, 64, 64, 8, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_small(None, None, None, 64, 64, 64, 16, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_small(None, None, None, 1 << 16, 64, 1 << 14, 32, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_small(None, None, None, 64, 0, 64, 32, None) == 0
    # streams and recorded launch sequences: NULL handles
    assert L.sgpu_stream_create(None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_stream_destroy(None) == 0
    assert L.sgpu_graph_begin(None) == sg.SGPU_ERR_INVALID_ARG      # the null stream cannot record
    assert L.sgpu_graph_end(None, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_graph_launch(None, None) == sg.SGPU_ERR_INVALID_ARG
    assert L.sgpu_graph_destroy(None) == 0


def test_gemv_multi_geometry_follows_the_token_rule(sg):
    """The matrix-core path (one 256-thread block per 32-token x 32-row tile) from T = 4, and
    from T = 9 once K > 1024; below that a wave per row (gemm_nt_ok in gemv_core.h)."""
    import ctypes as ct

    L = sg.lib()
    g, b = (ct.c_uint * 3)(), (ct.c_uint * 3)()
    for T, K, mfma in [(3, 768, False), (4, 768, True), (8, 1028, False), (9, 1028, True), (8, 1024, True)]:
        assert L.sgpu_kernel_geometry(b"gemv_multi", T, 2304, K, g, b) == 0
        assert b[0] == 256
        if mfma:
            assert (g[0], g[1]) == (((T + 31) // 32) * (2304 // 32), 1), (T, K)
        else:
            assert g[0] == 2304 // 4 and g[1] == (T + 15) // 16, (T, K)


def test_error_strings(sg):
    for code in (0, -1, -2, -3, -4, -5, -99):
        assert isinstance(sg.error_string(code), str) and sg.error_string(code)


def test_no_device_here_fails_loudly(sg):
    """Without a GPU the product path reports an error; it never computes on the CPU."""
    import sgpu

    if sgpu.lib().sgpu_init(0) == 0:
        pytest.skip("a device is present")
    A = np.ones(4, np.float32)
    with pytest.raises(sgpu.SgpuError):
        sgpu.DeviceArray.from_host(A)


def test_qwen_cfg_defaults(sg):
    c = sg.qwen_default_cfg()
    assert (c.V, c.C, c.NL, c.NH, c.NKV, c.HD, c.FC, c.CTX) == (151936, 896, 24, 14, 2, 64, 4864, 8192)
    assert abs(c.eps - 1e-6) < 1e-12 and c.theta == 1e6
