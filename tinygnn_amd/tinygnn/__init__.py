"""tinygnn -- the reference's Python package surface (python/tinygnn/__init__.py
of the reference) on the MI355X path.

The names are those of the reference's package, re-exported from this
build's ``_tinygnn_core`` module (``tinygnn_amd/_build``), whose tensors
live in HBM.  Put ``tinygnn_amd`` on ``sys.path`` (or PYTHONPATH) and
``import tinygnn`` works as with the reference.

Added for the device: :func:`to_torch` / :func:`from_torch` move data
between a Dense ``Tensor`` and a torch device tensor without a host round
trip (``to_torch`` is zero-copy through ``__cuda_array_interface__``).
"""
from __future__ import annotations

import os
import sys

_BUILD = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_build")
if _BUILD not in sys.path:
    sys.path.insert(0, _BUILD)

from _tinygnn_core import (  # noqa: E402
    Activation,
    CoraData,
    GATLayer,
    GCNLayer,
    GraphData,
    GraphLoader,
    Model,
    SAGELayer,
    StorageFormat,
    Tensor,
    WeightFile,
    add_bias,
    add_self_loops,
    edge_softmax,
    elu_inplace,
    gcn_norm,
    gelu_inplace,
    get_max_threads,
    leaky_relu_inplace,
    load_cora_binary,
    load_weight_file,
    log_softmax_inplace,
    matmul,
    relu_inplace,
    sage_max_aggregate,
    set_num_threads,
    sigmoid_inplace,
    softmax_inplace,
    spmm,
    tanh_inplace,
)

__all__ = [
    "StorageFormat", "Activation", "Tensor", "matmul", "spmm", "relu_inplace",
    "leaky_relu_inplace", "elu_inplace", "sigmoid_inplace", "tanh_inplace", "gelu_inplace",
    "softmax_inplace", "log_softmax_inplace", "add_bias", "add_self_loops", "gcn_norm",
    "edge_softmax", "sage_max_aggregate", "GCNLayer", "SAGELayer", "GATLayer", "Model",
    "CoraData", "WeightFile", "load_cora_binary", "load_weight_file", "GraphData", "GraphLoader",
    "set_num_threads", "get_max_threads", "to_torch", "from_torch",
]


class _Buffer:
    """Holds one CUDA-array-interface description and the tensor it views."""

    def __init__(self, owner, iface):
        self._owner = owner
        self.__cuda_array_interface__ = iface


def to_torch(t: Tensor):
    """A torch view of the tensor's HBM buffer (no copy): a [rows x cols]
    float32 tensor for Dense, (row_ptr, col_ind, values) for SparseCSR.  The
    view keeps ``t`` alive."""
    import torch
    dev = torch.device("cuda", torch.cuda.current_device())
    if t.format == StorageFormat.Dense:
        return torch.as_tensor(_Buffer(t, t.__cuda_array_interface__), device=dev)
    return tuple(torch.as_tensor(_Buffer(t, d), device=dev) for d in t.device_arrays())


def from_torch(x) -> Tensor:
    """A Dense Tensor holding a copy of a 2-D float tensor (device to device
    when ``x`` is on the GPU)."""
    import torch
    if x.dim() != 2:
        raise ValueError(f"from_torch: expected a 2-D tensor, got {x.dim()}-D")
    x = x.to(torch.float32).contiguous()
    if not x.is_cuda:
        return Tensor.from_numpy(x.numpy())
    torch.cuda.synchronize(x.device)
    return Tensor._from_device(x.shape[0], x.shape[1], x.data_ptr())


__version__ = "0.1.5"
