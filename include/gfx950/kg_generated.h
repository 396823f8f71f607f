/*
 * gfx950/kg_generated.h - entry points every generated per-operation kernel.hip defines
 * (gen_kernel/per_op.py). The fused form defines kg_execute_entry only.
 */
#pragma once

#include "kg_gfx950.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * The reference's entry of a generated shared object: slots in DSL parameter order
 * (kernel_gen/execute_engine/builtin_strategy/common.py:915-925, runtime_args.py:793-811).
 * The per-operation form allocates its workspace (one slice per workgroup for the
 * kernel's tiles, plus an error word) stream-ordered on the launch stream and frees it
 * after the launch. The kernel sets the error word when an operation addresses memory
 * outside a view; the entry reads it back (and returns -1) only in synchronous mode
 * (kg_gfx950_set_launch_mode): after an enqueue-only call such an error is not reported.
 */
int kg_execute_entry(const KgArgSlot* ordered_args, unsigned long long arg_count);

/*
 * No counterpart in the reference. For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * kg_execute_entry with the workspace taken from a fixed __device__ array of the generated
 * library instead of hipMallocAsync: exactly the largest grid's slices plus the error
 * word when every allocation of the kernel has a constant extent, else 32 MiB, held per
 * GPU for the life of the process. It runs the same kernel, on fewer workgroups when the
 * scratch cannot hold a slice for each, and so gives the same bits.
 * Returns -3 when one workgroup's workspace exceeds the scratch. Calls allocate nothing
 * (no hipMalloc, hipFree or allocating library routine); every call on a GPU shares that
 * GPU's scratch, so calls that overlap on one GPU race.
 */
int kg_execute_entry_noalloc(const KgArgSlot* ordered_args, unsigned long long arg_count);

#ifdef __cplusplus
}
#endif
