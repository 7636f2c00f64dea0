/* code_objects.S -- embeds the gfx950 code objects into libswitchgpu.so as read-only data.
 * The .co files are found on the assembler include path (-Wa,-I<build dir>). */
#define EMBED(sym, file)              \
    .section .rodata.sgpu_co, "a";    \
    .balign 4096;                     \
    .global sym;                      \
    .type sym, @object;               \
sym:                                  \
    .incbin file;                     \
    .global sym##_end;                \
sym##_end:                            \
    .byte 0

EMBED(sgpu_co_switch_gpu, "switch_gpu.co")
EMBED(sgpu_co_gemv, "gemv.co")
EMBED(sgpu_co_gpt2_kernels, "gpt2_kernels.co")
EMBED(sgpu_co_qwen_kernels, "qwen_kernels.co")
EMBED(sgpu_co_sgpu_tuned, "sgpu_tuned.co")
EMBED(sgpu_co_sgpu_decode, "sgpu_decode.co")
EMBED(sgpu_co_sgpu_probe, "sgpu_probe.co")

.section .note.GNU-stack, "", @progbits
