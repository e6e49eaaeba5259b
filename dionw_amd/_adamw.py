"""The AdamW route on the multi-tensor HIP kernel.

Reference: src/dionw/_adamw.py:18-61 (``torch._fused_adamw_`` with a float32
0-d device step counter per parameter). The step counters are incremented on
the device by one launch, then one launch per 48 tensors applies AdamW with
ATen's arithmetic, so results are bit-identical to torch's fused AdamW.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor

from dionw_amd import _lib
from dionw_amd._keys import ADAMW_STEP_STATE, EXP_AVG_SQ_STATE, EXP_AVG_STATE, ParamState
from dionw_amd._layout import same_dense_layout
from dionw_amd.ema._fusion import ACTIVE_EMA

__all__ = ["adamw_step", "init_adamw_state"]


def init_adamw_state(param: Tensor, state: dict[str, Any]) -> None:
    """Fresh AdamW moments and step counter in ``state``."""
    state.update({
        EXP_AVG_STATE: torch.zeros_like(param),
        EXP_AVG_SQ_STATE: torch.zeros_like(param),
        # a 0-d float32 tensor on the parameter's device, as torch's fused AdamW takes it
        ADAMW_STEP_STATE: param.new_zeros((), dtype=torch.float32),
    })


def adamw_step(group: dict[str, Any], state: ParamState) -> None:
    """One AdamW step of the group's parameters that have gradients.

    Raises:
        RuntimeError: If a parameter chosen for the pass has lost its gradient.
        TypeError: For a parameter that is not float32.
    """
    params = [p for p in group["params"] if p.grad is not None]
    if not params:
        return
    entries = [state[p] for p in params]
    targets: list[Tensor] = []
    grads: list[Tensor] = []
    exp_avgs: list[Tensor] = []
    exp_avg_sqs: list[Tensor] = []
    copies: list[tuple[Tensor, Tensor]] = []
    for param, entry in zip(params, entries, strict=True):
        if EXP_AVG_STATE not in entry:
            init_adamw_state(param, entry)
        grad = param.grad
        if grad is None:
            raise RuntimeError("every parameter of an AdamW pass needs a gradient")
        if param.dtype != torch.float32:
            raise TypeError(f"the HIP AdamW takes float32 parameters, got {param.dtype}")
        data = param.data
        m, v = entry[EXP_AVG_STATE], entry[EXP_AVG_SQ_STATE]
        grad = grad.to(torch.float32)
        if not all(same_dense_layout(t, data) for t in (grad, m, v)):
            # Mixed layouts: step row-major copies and write them back.
            flat = [t.contiguous() for t in (data, m, v)]
            copies.extend(zip((data, m, v), flat, strict=True))
            data, m, v = flat
            grad = grad.contiguous()
        targets.append(data)
        grads.append(grad)
        exp_avgs.append(m)
        exp_avg_sqs.append(v)
    steps = [entry[ADAMW_STEP_STATE] for entry in entries]
    stream = _lib.stream_handle(params[0].device)
    _lib.call("dionw_increment_steps", _lib.ptr_array(steps), len(steps), stream)
    beta1, beta2 = group["betas"]
    tensors = (_lib.ptr_array(targets), _lib.ptr_array(grads), _lib.ptr_array(exp_avgs),
               _lib.ptr_array(exp_avg_sqs), _lib.ptr_array(steps))
    sizes = (_lib.int64_array([t.numel() for t in targets]), len(targets))
    scalars = (float(group["lr"]), float(beta1), float(beta2), float(group["weight_decay"]),
               float(group["eps"]))
    # A due GPU EMA lerp of these parameters rides on the AdamW pass.
    ema = ACTIVE_EMA.get()
    shadows = ema.fusable_shadows(params) if ema is not None and not copies else None
    if shadows is None:
        _lib.call("dionw_adamw", *tensors, *sizes, *scalars, stream)
    else:
        _lib.call("dionw_adamw_ema", *tensors, _lib.ptr_array(shadows), *sizes, *scalars,
                  ema.fused_weight(), stream)
        ema.mark_fused(params)
    for original, copy in copies:
        if original.data_ptr() != copy.data_ptr():
            original.copy_(copy)
    if ema is not None:
        ema.stage_written(params)
