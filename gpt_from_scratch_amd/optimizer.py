"""The train step's optimizer with its AdamW step in two HIP kernels.

Drop-in for ``core/optimizer.py``'s ``DistributedOptimizer`` at one
data-parallel rank, constructed and called the same way (train.py:130-139,
:172, :187)::

    optimizer = DistributedOptimizer(model, optimizer_cls=torch.optim.AdamW,
                                     optimizer_kwargs={"lr": 3e-4, "weight_decay": 0.1,
                                                       "betas": (0.9, 0.95)},
                                     clip_grad=1.0)
    optimizer.zero_grad(); loss.backward(); optimizer.step()

As in the reference, the parameters and gradients are re-pointed into flat
bf16 buffers the model computes in, and an fp32 master copy takes the update.
With ``torch.optim.AdamW`` the step is:

* ``mi_grad_sumsq``: the squared gradient norm, reduced on the device in a
  fixed order;
* ``mi_adamw_step``: one pass over the flat buffers that applies the clip
  (read from device memory: no host synchronisation, where the reference
  compares the norm on the host), the AdamW update of the fp32 master and
  moments, and the copy back into the bf16 parameter buffer.

The reference instead converts the gradient buffer to an fp32 copy, runs
torch's multi-tensor AdamW (several passes over the master and the moments)
and converts the master back.  Any other ``optimizer_cls`` runs the
reference's own sequence on torch's optimizer (on the GPU: parameters
elsewhere are refused, as by every operator of this package).

The moments live in ``self.optimizer.state`` under torch's names, so
``state_dict()`` / ``load_state_dict()`` read and write torch's AdamW format,
and the hyperparameters are read from ``self.optimizer.param_groups`` at every
step (a learning-rate schedule that edits them works as with torch).
"""
from __future__ import annotations

import torch

from . import _lib


def _data_parallel_world_size() -> int:
    import torch.distributed as dist
    if dist.is_available() and dist.is_initialized():
        return dist.get_world_size()
    return 1


class DistributedOptimizer:
    def __init__(self, model: torch.nn.Module, optimizer_cls, optimizer_kwargs: dict,
                 clip_grad: float = 1.0, dtype: torch.dtype = torch.bfloat16):
        if _data_parallel_world_size() != 1:
            raise NotImplementedError(
                "this build runs one data-parallel rank per job (one GPU); the gradient "
                "reduce-scatter / parameter all-gather of core/optimizer.py:81,95 are not built")
        self.model = model
        self.optimizer_kwargs = optimizer_kwargs
        self.clip_grad = clip_grad
        self.dtype = dtype
        self.params = [p for p in model.parameters() if p.requires_grad]
        _lib._require_gpu(*self.params)
        total = sum(p.numel() for p in self.params)
        self.padding_size = 0
        self.padded_numel = total
        self.shard_size = total
        dev = self.params[0].device
        self.param_buffer = torch.zeros(total, dtype=dtype, device=dev)
        self.grad_buffer = torch.zeros(total, dtype=dtype, device=dev)
        offset = 0
        for p in self.params:
            k = p.numel()
            self.param_buffer[offset:offset + k].copy_(p.data.view(-1))
            p.data = self.param_buffer[offset:offset + k].view(p.shape)
            p.grad = self.grad_buffer[offset:offset + k].view(p.shape)
            offset += k
        self.fp32_master_shard = (self.param_buffer.to(torch.float32).clone().detach()
                                  .requires_grad_(True))
        self.optimizer = optimizer_cls([self.fp32_master_shard], **optimizer_kwargs)
        self.fused = optimizer_cls is torch.optim.AdamW and self._fusable()
        self._ws = None
        self._norm_valid = False

    def _fusable(self) -> bool:
        g = self.optimizer.param_groups[0]
        # the fused step keeps torch's default (non-capturable) state layout
        return (not g.get("amsgrad", False) and not g.get("maximize", False)
                and not g.get("capturable", False) and not g.get("differentiable", False))

    def zero_grad(self):
        """Clear the gradient buffer (never set grads to None: they point into it)."""
        self.grad_buffer.zero_()

    def step(self):
        if not self.fused:
            return self._step_reference()
        _lib._require_gpu(self.grad_buffer)
        if self._ws is None:
            self._ws = torch.empty(_lib.adamw_workspace(), dtype=torch.float32,
                                   device=self.grad_buffer.device)
        group = self.optimizer.param_groups[0]
        master = self.fp32_master_shard
        state = self.optimizer.state[master]
        if len(state) == 0:
            # torch.optim.AdamW's lazy state: a CPU step counter and zero moments
            state["step"] = torch.tensor(0.0, dtype=torch.float32)
            state["exp_avg"] = torch.zeros_like(master, memory_format=torch.preserve_format)
            state["exp_avg_sq"] = torch.zeros_like(master, memory_format=torch.preserve_format)
        state["step"] += 1
        t = float(state["step"])
        lr = float(group["lr"])
        beta1, beta2 = (float(b) for b in group["betas"])
        # the host-side scalars torch's multi-tensor AdamW computes in Python floats
        bc1 = 1 - beta1 ** t
        bc2 = 1 - beta2 ** t
        hp = (1 - lr * float(group["weight_decay"]), 1 - beta1, beta2, 1 - beta2, lr / bc1,
              bc2 ** 0.5, float(group["eps"]), float(self.clip_grad or 0.0))
        clip = self.clip_grad is not None and self.clip_grad > 0.0
        if clip:
            _lib.grad_sumsq(self.grad_buffer, self._ws)
        self._norm_valid = clip
        _lib.adamw_step(self.grad_buffer, master.data, state["exp_avg"], state["exp_avg_sq"],
                        self.param_buffer, hp, self._ws if clip else None)

    def _step_reference(self):
        """core/optimizer.py:79-104 at one rank, on torch's optimizer: other optimizer
        classes, and AdamW variants the fused step does not cover (amsgrad, maximize,
        capturable, differentiable)."""
        self._norm_valid = False
        reduced = self.grad_buffer.clone()
        if self.clip_grad is not None and self.clip_grad > 0.0:
            norm = torch.sqrt(torch.sum(reduced.to(torch.float32) ** 2))
            if norm > self.clip_grad:
                reduced.mul_(self.clip_grad / (norm + 1e-6))
        self.fp32_master_shard.grad = reduced.to(self.fp32_master_shard.dtype)
        self.optimizer.step()
        self.optimizer.zero_grad()
        self.param_buffer.copy_(self.fp32_master_shard.detach().to(self.dtype))

    def grad_norm(self) -> torch.Tensor:
        """The global gradient norm of the last fused step (a device tensor), as
        clipped against.  Only computed when clipping is on."""
        if not self._norm_valid:
            raise RuntimeError("no fused step with clipping has run")
        return torch.sqrt(self._ws[0])

    def state_dict(self):
        return self.optimizer.state_dict()

    def load_state_dict(self, state_dict):
        self.optimizer.load_state_dict(state_dict)
