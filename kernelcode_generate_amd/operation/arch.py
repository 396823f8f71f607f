"""Launch queries of the DSL (kernel_gen/operation/arch.py:652-776): `get_block_id()`,
`get_block_num()`, `get_thread_id()`, `get_thread_num()`, `get_subthread_id()`,
`get_subthread_num()`. Inside a kernel each is a symbolic integer of the launch."""

from __future__ import annotations

from ._marker import dsl_op

get_block_id = dsl_op("arch.get_block_id")
get_block_num = dsl_op("arch.get_block_num")
get_thread_id = dsl_op("arch.get_thread_id")
get_thread_num = dsl_op("arch.get_thread_num")
get_subthread_id = dsl_op("arch.get_subthread_id")
get_subthread_num = dsl_op("arch.get_subthread_num")

__all__ = ["get_block_id", "get_block_num", "get_subthread_id", "get_subthread_num", "get_thread_id",
           "get_thread_num"]
