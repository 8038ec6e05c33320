// nes_step_full.hip -- the step kernel's all-RAM-in-LDS instances (batches
// whose consoles' 2 KB of RAM all fit in LDS: up to 8,192 consoles), built
// from nes_step.hip in a translation unit of their own so that they take a
// scheduler flag of their own (nesle_amd/build.py).  With LLVM's iterative
// ILP scheduler these instances run 2-3 % faster (4,096 consoles: 14.22 ->
// 13.85 ms per launch, 8,192: 14.61 -> 14.31), and about 1 % more with the
// scheduler's macro-op fusion off; the split-layout instances at 64 consoles
// per wave run 2.5 % slower with the ILP scheduler (65,536 consoles).
#define NESLE_STEP_PART 1
#include "nes_step.hip"
