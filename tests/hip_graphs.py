"""Helper for the compile tests: HIP graphs recorded by inductor's cudagraph
trees (torch.compile mode="reduce-overhead") on the current device."""

from __future__ import annotations

import torch


def recorded_hip_graphs() -> int:
    from torch._inductor import cudagraph_trees

    mgr = cudagraph_trees.get_manager(torch.cuda.current_device(), create_if_none_exists=False)
    if mgr is None or mgr.roots is None:
        return 0
    n, stack = 0, [node for roots in mgr.roots.values() for node in roots]
    while stack:
        node = stack.pop()
        n += 1
        stack.extend(c for children in node.children.values() for c in children)
    return n


def reset() -> None:
    """Forget compiled code and every recorded graph (count from zero)."""
    from torch._inductor.cudagraph_trees import reset_cudagraph_trees

    torch._dynamo.reset()
    reset_cudagraph_trees()
