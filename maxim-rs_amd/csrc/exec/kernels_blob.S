/* The gfx950 code object, embedded in the library the way the reference
 * embeds its fatbins (src/cuda.rs, include_bytes!). */
    .section .rodata
    .global mx_kernels_hsaco
    .global mx_kernels_hsaco_end
    .p2align 12
mx_kernels_hsaco:
    .incbin HSACO_PATH
mx_kernels_hsaco_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
