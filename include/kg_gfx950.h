/*
 * kg_gfx950.h - C ABI of the MI355X (gfx950) backend for kernelcode_generate's
 * data-parallel hot path: the tiled matmul, conv2d and flash-attention demo kernels.
 *
 * Every compute entry point has exactly the signature of the entry that the
 * reference's execute engine binds through ctypes in a generated shared object:
 *
 *     extern "C" int kg_execute_entry(const _ArgSlot* ordered_args,
 *                                     unsigned long long arg_count);
 *
 *   reference: kernel_gen/execute_engine/builtin_strategy/common.py:915-925 (C++ shim),
 *              kernel_gen/execute_engine/runtime_args.py:217-237 (_CArgSlot, ctypes),
 *              kernel_gen/execute_engine/runtime_args.py:793-811 (invoke_compiled_kernel)
 *
 * A gfx950 generated source (SourceBundle kernel.hip) defines kg_execute_entry as a
 * forward to one of the entries below, so the reference's CompiledKernel.execute()
 * contract (slots in DSL parameter order, return 0 on success, non-zero ->
 * "runtime_throw_or_abort") is unchanged.
 *
 * Memory slots carry DEVICE pointers (torch ROCm tensor .data_ptr()), element shapes
 * and element strides. Kernels allocate nothing per call, with one exception: matmul and
 * conv2d calls that split K over workgroups keep their fp32 partial sums in a workspace
 * held per (device, stream) for the life of the process, allocated on the first such call
 * on that stream and reallocated when a later one needs more. Those calls are therefore
 * not safe under HIP graph capture unless an earlier call of at least the same size ran on
 * that stream uncaptured. Calls are synchronous by default (the reference's cuda_sm89
 * launch ends with a device synchronize, include/cuda_sm89/Arch.h:166-168);
 * kg_gfx950_set_launch_mode() switches to asynchronous launches on a caller-chosen stream
 * for benchmarking.
 *
 * Return codes: 0 ok; -1 slot/shape/dtype validation failure; -2 HIP runtime error;
 * -3 unsupported configuration. kg_gfx950_last_error() describes the last failure.
 */
#ifndef KG_GFX950_H_
#define KG_GFX950_H_

#ifdef __cplusplus
extern "C" {
#endif

/* Slot kinds: reference builtin_strategy/common.py:910-914 (KG_ARG_MEMORY/INT/FLOAT). */
enum {
  KG_ARG_MEMORY = 1,
  KG_ARG_INT = 2,
  KG_ARG_FLOAT = 3
};

/* dtype codes 1-4 are the reference's (runtime_args.py:94-110, common.py:171-194);
 * 5 (float16) and 6 (bfloat16) are additive extensions for the gfx950 MFMA paths. */
enum {
  KG_DTYPE_F32 = 1,
  KG_DTYPE_F64 = 2,
  KG_DTYPE_I32 = 3,
  KG_DTYPE_I64 = 4,
  KG_DTYPE_F16 = 5,
  KG_DTYPE_BF16 = 6
};

/* Byte-for-byte the reference's _ArgSlot / _CArgSlot (runtime_args.py:228-237;
 * common.py:915-924; include/cuda_sm89/Core.h:156-165). 64 bytes on LP64. */
typedef struct KgArgSlot {
  int kind;
  void* data;
  const long long* shape;
  const long long* stride;
  unsigned long long rank;
  int dtype_code;
  long long int_value;
  double float_value;
} KgArgSlot;

/*
 * Matmul demos: kernel/matmul/inputs_static_tile_static.py:56-110,
 * kernel/matmul/inputs_static_tile_dynamic.py:64-120,
 * kernel/matmul/inputs_dynamic_tile_dynamic.py:57-113.
 * Slot order (test/cuda/test_cuda_sm89_kernel_demos_runtime.py:520):
 *   (out[M,N], lhs[M,K], rhs[K,N], bias[N] | absent [, tile_m, tile_n, tile_k [, memory_stage]])
 * 4, 7 or 8 slots. dtypes: all f32, all bf16 or all f16 (bias may be f32 with bf16/f16
 * operands). Absent bias = memory slot with data == NULL (runtime_args.py:497-516).
 * Result: out = lhs @ rhs (+ bias[None, :]), fp32 accumulation. Slot 7 is an additive
 * extension: INT memory_stage in {2, 3, 4}, the LDS ring depth of the pipelined 16-bit
 * kernel (the gfx950 reading of the reference's multi-buffer memory_stage,
 * kernel_gen/passes/memory/multi_buffer.py; default 4); other kernels ignore it.
 * 16-bit outputs of at most 64 tiles of 128 x 256 with K >= 512 split K over workgroups and
 * add the fp32 partial sums in a second kernel; the partials live in a workspace the library
 * allocates once per (device, stream) on first use (hipMalloc, at most 64 MiB) and keeps.
 */
int kg_gfx950_matmul_entry(const KgArgSlot* ordered_args, unsigned long long arg_count);

/*
 * Conv2d demos (NCHW): kernel/conv2d/inputs_static_tile_static.py:115-215,
 * kernel/conv2d/inputs_static_tile_dynamic.py:120, kernel/conv2d/inputs_dynamic_tile_dynamic.py:102-205.
 * Slot order is the dynamic demo's (test/cuda/test_cuda_sm89_kernel_demos_runtime.py:380-404):
 *   (out[N,F,Ho,Wo], input[N,C,H,W], weight[F,C,KH,KW], bias[F] | absent,
 *    stride_h, stride_w, dilation_h, dilation_w, pad_top, pad_bottom, pad_left, pad_right
 *    [, tile_f, tile_c, tile_n, tile_ho, tile_wo])
 * 12 or 17 slots. Static demos bake stride/dilation/pad into their generated entry,
 * which forwards the constants here. Ho/Wo follow kernel/conv2d/inputs_static_tile_static.py:155-156.
 * 16-bit and fp32 convs whose grid would leave CUs idle (small batches, deep 14x14 / 7x7
 * layers) split the contraction over workgroups and add the fp32 partial sums in a second
 * kernel, in the matmul's per-(device, stream) workspace (allocated on first use, kept).
 */
int kg_gfx950_conv2d_entry(const KgArgSlot* ordered_args, unsigned long long arg_count);

/*
 * Flash-attention forward demos: kernel/flash_attention/inputs_static_tile_static.py:90-190,
 * .../inputs_static_tile_dynamic.py:96, .../inputs_dynamic_tile_dynamic.py:96-195.
 * Slot order (test/cuda/test_cuda_sm89_kernel_demos_runtime.py:592):
 *   (out[B,H,S,D], q[B,H,S,D], k[B,H,S,D], v[B,H,S,D] [, br, bc [, scale, causal]])
 * 4, 6 or 8 slots. The reference computes softmax(Q K^T) V with no scale and no mask;
 * slots 6-7 are an additive extension: FLOAT scale (default 1.0) and INT causal
 * (0/1, lower-triangular mask including the diagonal).
 */
int kg_gfx950_flash_attention_entry(const KgArgSlot* ordered_args, unsigned long long arg_count);

/*
 * Launch control (no counterpart in the reference, whose execute() is synchronous and
 * rejects a stream: compiler.py:286-291). synchronous != 0 (default): every entry
 * synchronizes its stream before returning. synchronous == 0: entries only enqueue on
 * `stream` (a hipStream_t; NULL = null stream). Returns 0.
 */
int kg_gfx950_set_launch_mode(int synchronous, void* stream);

/*
 * Support for generated entries (no counterpart in the reference, whose generated sources
 * include their runtime headers; here the runtime is this library). A generated
 * kg_execute_entry (the gfx950 emitter's kernel.hip) validates its slots, launches on the
 * calling thread's stream and reports failures through these, so the execute engine
 * reads one error text per thread whichever code failed.
 *
 * kg_gfx950_fail: records `message` as the calling thread's last error; returns `code`.
 * kg_gfx950_check_memory_slot: slot `index` must be a memory slot of rank `rank` holding
 *   a device pointer whose strided view fits its allocation (the entries' own check);
 *   allow_absent != 0 accepts data == NULL; dtype_code != 0 must equal the slot's. 0 or -1.
 * kg_gfx950_launch_stream / kg_gfx950_launch_synchronous: the calling thread's launch mode
 *   (kg_gfx950_set_launch_mode).
 * kg_gfx950_finish_launch: checks the last launch and, in synchronous mode, waits for the
 *   stream; 0, or -2 with the HIP error recorded.
 */
int kg_gfx950_fail(int code, const char* message);
int kg_gfx950_check_memory_slot(const KgArgSlot* slots, int index, int rank, int allow_absent, int dtype_code,
                                const char* name);
void* kg_gfx950_launch_stream(void);
int kg_gfx950_launch_synchronous(void);
int kg_gfx950_finish_launch(const char* what);

/* Text of the last failure on the calling thread ("" if none). */
const char* kg_gfx950_last_error(void);

/* ABI revision of this library (bumped on any change of a declaration here or of the slot
 * contract). 2: kg_gfx950_cost writes five kinds (KG_COST_MFMA_CYCLES added). 3: the
 * measurement aid kg_gfx950_mfma_rate left the library (bench.py's probe library has it);
 * memory_stage slots on the attention (slot 8) and conv2d (slot 17) entries. */
int kg_gfx950_abi_version(void);

/* Operations and cost kinds of kg_gfx950_cost. */
enum {
  KG_OP_MATMUL = 1,
  KG_OP_CONV2D = 2,
  KG_OP_FLASH_ATTENTION = 3
};
enum {
  KG_COST_MAC = 0,       /* multiply-accumulates of the operation (mask-kept pairs for causal attention) */
  KG_COST_MFMA = 1,      /* wave-level MFMA instructions the chosen kernel issues (0 on SIMT paths) */
  KG_COST_HBM_READ = 2,  /* compulsory bytes read: every input element once */
  KG_COST_HBM_WRITE = 3, /* compulsory bytes written: every output element once */
  KG_COST_MFMA_CYCLES = 4, /* SIMD cycles those MFMA instructions occupy (shapes differ per kernel) */
  KG_COST_KINDS = 5
};

/*
 * Static cost of one call, without a GPU: replaces the reference's dsl_cost_run
 * (kernel_gen/tools/dsl_run.py:656-730), which runs the npu_demo cost pipeline and
 * returns one integer per cost kind (DMA1..DMA4, MAC, VECTOR1, VECTOR2). op is a
 * KG_OP_* code; ordered_args/arg_count are exactly the slots the matching entry above
 * takes (memory slots need shapes, strides and dtypes; a non-NULL data pointer marks a
 * present operand and is never dereferenced). The entry's own validation and kernel choice run unchanged, so a call the
 * entry would reject fails here with the same code and message. On success writes
 * KG_COST_KINDS values to costs[] and returns 0.
 */
int kg_gfx950_cost(int op, const KgArgSlot* ordered_args, unsigned long long arg_count, long long* costs);

#ifdef __cplusplus
}
#endif

#endif /* KG_GFX950_H_ */
