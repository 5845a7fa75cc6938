"""zeromoe_amd -- MI355X (gfx950) routed-expert MUL_MAT_ID path.

Host mirror of the reference's operator surface over the C ABI of
libzeromoe_hip.so (include/zeromoe.h):

* :func:`mul_mat_id` -- ``ggml_mul_mat_id`` semantics on device tensors
  (/root/reference/models/graph/moe_routed_ggml.hpp:172-193).
* :func:`router` -- ``moe_routed::gate_probs/select_ids/route_weights``
  (moe_routed_ggml.hpp:52-141) with the slot table of
  ``make_branch_inputs`` (backends/ggml/moe_partial_route_ggml.hpp:21-35).
* :func:`bucket` -- the per-expert CSR of core/batched_dispatch_pipeline.cpp:1181-1202.
* :class:`MoELayer` -- one routed layer (expert_ffn + weighted sum_topk +
  shared expert, moe_routed_ggml.hpp:166-214, moe_block.hpp:86-105).
* FP32-activation path of the CUDA executor: :func:`f32_matmul`
  (launch_<type>_matmul, kernels/quant/kquant_matmul.cu:575-599),
  :func:`mul_mat_id_f32` (native_f32_quant_hook, kquant_matmul.cu:702-756),
  :func:`swiglu`, :func:`scatter_accum`, :func:`glm5next_router_topk`
  (kernels/math/expert_activation.cu, expert_accum.cu,
  kernels/models/glm5next_router.cu) and :class:`ExpertExecutor`
  (core/gpu_expert_executor.hpp:42-58).
* :func:`moe_unpack` -- expert-major [gate|up|down] transfer records to the
  planar expert tensors (launch_ggml_moe_unpack[_scatter],
  kernels/math/ggml_moe_pack.cu:127-179).

Torch is used only for device memory and the current stream.
"""
from __future__ import annotations

from .ops import (GGML_TYPES, ColdLane, ExpertExecutor, MoELayer, block_dots, bucket, builtin_iq2xxs_grid, builtin_iq3xxs_grid,
                  builtin_iq4nl_table,                   f32_matmul,
                  glm5next_router_topk, init, moe_unpack, mul_mat_id, mul_mat_id_f32, quantize_q8_K, router, row_size,
                  scatter_accum, set_iq2xxs_grid, set_iq3xxs_grid, set_iq4nl_table, swiglu)

__all__ = ["GGML_TYPES", "ColdLane", "ExpertExecutor", "MoELayer", "block_dots", "bucket", "builtin_iq2xxs_grid", "builtin_iq3xxs_grid", "builtin_iq4nl_table",
           "f32_matmul",
           "glm5next_router_topk", "init", "moe_unpack", "mul_mat_id", "mul_mat_id_f32", "quantize_q8_K", "router", "row_size",
           "scatter_accum", "set_iq2xxs_grid", "set_iq3xxs_grid", "set_iq4nl_table", "swiglu"]
