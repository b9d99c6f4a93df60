"""Host-side front end of the HIP realizer: the reference JIT's realize path.

ir          UOp IR (_ir.py)
tensor      graph building with the reference's op semantics (_tensor_proxy.py,
            _functional.py, _amp.autocast)
amp         cast insertion (_amp.insert_cast_pass)
fusion      elementwise-chain / softmax fusion (_fusion.fuse)
hip_fusion  this build's subgraph -> single-kernel rewrites
gpu_plan    tensor-plan builder (_gpu_plan.py)
buffers     BufferTable / GpuBufferTable (_buffer_table.py, _gpu_buffer_table.py)
realize     the walker and the plan route (_realize_webgpu.py)
configs     the benchmark graphs C1-C5 with their synthetic inputs
"""
from .buffers import BufferTable, GpuBufferTable
from .ir import UOp, toposort
from .realize import (
    RealizationError, get_registered_bridge, get_registered_gpu_buffer_table, is_available, materialize_gpu_buffer,
    realize_hip, realize_tensor_plan_hip, realize_tensor_plan_hip_resident, register_hip_bridge,
    supported_opcodes, unregister_hip_bridge,
)
from .tensor import Session, Tensor, autocast

__all__ = [
    "BufferTable", "GpuBufferTable", "UOp", "toposort", "Session", "Tensor", "autocast", "RealizationError",
    "realize_hip", "realize_tensor_plan_hip", "realize_tensor_plan_hip_resident", "materialize_gpu_buffer",
    "register_hip_bridge", "unregister_hip_bridge", "get_registered_bridge", "get_registered_gpu_buffer_table",
    "is_available", "supported_opcodes",
]
