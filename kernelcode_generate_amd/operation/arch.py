"""`arch` operations of the DSL (kernel_gen/operation/arch.py): the launch queries
`get_block_id()`, `get_block_num()`, `get_thread_id()`, `get_thread_num()`,
`get_subthread_id()`, `get_subthread_num()` (:652-776; inside a kernel each is a symbolic
integer of the launch) and `barrier(visibility=, scope=)` (:803). `get_dynamic_memory`
(:778) and `launch_kernel` name operations the gfx950 front end rejects with an error."""

from __future__ import annotations

from ._marker import dsl_op

get_block_id = dsl_op("arch.get_block_id")
get_block_num = dsl_op("arch.get_block_num")
get_thread_id = dsl_op("arch.get_thread_id")
get_thread_num = dsl_op("arch.get_thread_num")
get_subthread_id = dsl_op("arch.get_subthread_id")
get_subthread_num = dsl_op("arch.get_subthread_num")
barrier = dsl_op("arch.barrier")
get_dynamic_memory = dsl_op("arch.get_dynamic_memory")
launch_kernel = dsl_op("arch.launch_kernel")

__all__ = ["barrier", "get_block_id", "get_block_num", "get_dynamic_memory", "get_subthread_id", "get_subthread_num",
           "get_thread_id", "get_thread_num", "launch_kernel"]
