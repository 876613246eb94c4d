/* Embeds the gfx950 code object built from kernels/vearo_kernels.hip into
 * libvearo_hip.so; the runtime hands these bytes to hipModuleLoadData. */
  .section .rodata.vh_code_object, "a", @progbits
  .balign 4096
  .globl vh_code_object_start
  .type vh_code_object_start, @object
vh_code_object_start:
  .incbin "vearo_kernels.co"
  .globl vh_code_object_end
vh_code_object_end:
  .byte 0
  .section .note.GNU-stack, "", @progbits
