/* Embeds the gfx950 code object built from csrc/kernels/all.hip. */
    .section .rodata.t0_hsaco, "a", @progbits
    .p2align 12
    .globl t0_hsaco_start
    .globl t0_hsaco_end
t0_hsaco_start:
    .incbin T0_HSACO_PATH
t0_hsaco_end:
    .byte 0
    .section .note.GNU-stack, "", @progbits
