// emu_swap(void** save_sp, void* load_sp): saves the callee-saved registers
// of the running context on its stack, stores its stack pointer in
// *save_sp, and resumes the context whose stack pointer is load_sp
// (x86-64 System V).  Used by the CPU emulation scheduler of tests/emu.
    .text
    .globl emu_swap
    .type emu_swap, @function
emu_swap:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
    .size emu_swap, .-emu_swap
    .section .note.GNU-stack,"",@progbits
