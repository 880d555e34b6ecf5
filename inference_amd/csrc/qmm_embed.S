/* Embeds the gfx950 code object (built by the Makefile) into libqmm.so. */
    .section .rodata
    .balign 4096
    .global qmm_code_object_start
    .type qmm_code_object_start, @object
qmm_code_object_start:
    .incbin "qmm_kernels.co"
    .global qmm_code_object_end
qmm_code_object_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
