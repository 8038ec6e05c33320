// nes_step_narrow.hip -- the step kernel's split-layout instances for 16 or
// 32 consoles per wave (8,193 to 32,768 consoles; the pixel workload runs
// 16,384), built from nes_step.hip in a translation unit of their own so
// that they take a scheduler flag of their own (nesle_amd/build.py).  With
// the machine scheduler off (the instruction order the selection DAG
// leaves) they run 2-3 % faster (16,384 consoles: 17.09 -> 16.66 ms per
// launch, 32,768: 17.68 -> 17.36); at 64 consoles per wave (65,536) the
// same setting runs 0.6 % slower, so nes_step.hip keeps the default there.
#define NESLE_STEP_PART 2
#include "nes_step.hip"
