// Prefill kernel instances for head dims 192 and 256: a second translation unit
// of prefill.hip, compiled (see build.py) with LLVM's iterative ILP machine
// scheduler, which runs these one-wave-per-SIMD instances 8-12% faster than
// the default scheduler.  It defines akt::prefill_launch_wide and no C entry
// point.
#define AKT_PREFILL_WIDE_TU 1
#include "prefill.hip"
