"""Module-tree helpers shared by the decoder wrappers."""
from __future__ import annotations

import copy

import torch


def share_containers(module, _seen=None):
    """A copy of a module tree whose containers are new and whose tensors are shared.

    Every submodule is copied once (a module reachable along two paths stays one module in the
    copy); parameter and buffer dictionaries are copied, the tensors in them are not.  Replacing
    a child of the copy leaves the source tree untouched."""
    seen = {} if _seen is None else _seen
    if id(module) not in seen:
        twin = copy.copy(module)
        seen[id(module)] = twin
        twin._parameters = dict(module._parameters)
        twin._buffers = dict(module._buffers)
        twin._modules = {name: child if child is None else share_containers(child, seen)
                         for name, child in module._modules.items()}
    return seen[id(module)]


def require_inference(module):
    """The INT8 decoder modules run in eval mode with autograd off."""
    if module.training or torch.is_grad_enabled():
        raise RuntimeError("eval + inference/no_grad required")
