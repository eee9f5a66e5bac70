/* Links the ahead-of-time gfx950 code object into libtiler_hip.so as bytes.
 * TILER_HSACO_PATH is the quoted path of the object hipcc/clang produced. */
    .section .rodata.tiler_hip_code_object,"a",@progbits
    .balign 4096
    .globl tiler_hip_code_object
    .type tiler_hip_code_object, @object
tiler_hip_code_object:
    .incbin TILER_HSACO_PATH
    .globl tiler_hip_code_object_end
tiler_hip_code_object_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
