/* Links the ahead-of-time gfx950 code object into libtiler_hip.so as bytes.
 * TILER_HSACO_PATH is the quoted path of the object clang produced. */
    .section .rodata.tiler_hip_code_object,"a",@progbits
    .balign 4096
    .globl tiler_hip_code_object
    .type tiler_hip_code_object, @object
tiler_hip_code_object:
    .incbin TILER_HSACO_PATH
    .globl tiler_hip_code_object_end
tiler_hip_code_object_end:
    .byte 0
/* The kernel sources the code object was compiled from, as the build's
 * canonical source bundle (TILER_SOURCE_BUNDLE_PATH). */
    .section .rodata.tiler_hip_source_bundle,"a",@progbits
    .balign 16
    .globl tiler_hip_source_bundle
    .type tiler_hip_source_bundle, @object
tiler_hip_source_bundle:
    .incbin TILER_SOURCE_BUNDLE_PATH
    .globl tiler_hip_source_bundle_end
tiler_hip_source_bundle_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
