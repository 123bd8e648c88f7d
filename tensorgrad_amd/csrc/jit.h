// Kernels generated per fused group and compiled at run time (hipRTC) for gfx950.
//
// A fused group's program (FusedProgram + FusedInstr[], the same description the
// interpreter in k_fused.hip executes) becomes straight-line HIP source: iteration
// sizes, operand strides and opcodes are compile-time constants, every value lives in
// VGPRs, all operand loads are issued before the arithmetic, and the per-opcode
// arithmetic is fused_dev.h's op_eval, so generated kernels and the interpreter produce
// the same bits. Kernels are named by a hash of their source; one process-wide cache
// compiles each distinct kernel once.
#pragma once
#include <string>
#include <vector>

#include "kernels.h"

namespace tgk {

struct JitKernel {
  std::string name;   // tg_<hash of body>
  std::string body;   // extern "C" __global__ definition
  int64_t grid = 0;   // blocks of 256 threads
  bool gemm = false;  // a GEMM with a fused epilogue (its program needs gemm_dev.h)
};

// Source of a GEMM kernel (gemm_dev.h's tile) whose epilogue runs the element program p
// (one element per call, vec = 1) on each product element instead of storing it.
JitKernel gemm_epi_kernel(const FusedProgram& p, const FusedInstr* code, const GemmEpiCfg& c);

// Source of the kernel for `p` (its code[] instructions) over n threads' runs (element
// form: elements / vec) or n rows (row form).
JitKernel fused_kernel(const FusedProgram& p, const FusedInstr* code, int64_t n);

// Compile every kernel of `ks` that is not compiled yet, in one hipRTC program. With
// load, also load the code objects on the current device. Throws std::runtime_error with
// the compiler log on failure.
void jit_compile(const std::vector<JitKernel>& ks, bool load);

// The loaded function of a compiled kernel on the current device.
hipFunction_t jit_function(const std::string& name);

}  // namespace tgk
