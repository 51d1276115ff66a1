"""Adam and AdamW over a GPT's parameters, stepped on the device
(NimbleML/optimizers/adam.py:44-311, optimizers/optimizer.py:5-100).

The constructor, ``param_groups``, ``t``, ``learning_rate`` / ``get_lr`` / ``set_lr`` and
``zero_grad`` are the reference's. ``step()`` pushes the host gradients that
``loss.backward()`` accumulated into the model's device gradient arena (skipped when the
arena already holds them: one backward since the gradients were cleared), then runs the
reference's float32 AdamW update (native/src/adamw.cpp:6-20 operation order) on the device:
one launch over the whole model when there is one parameter group and every parameter has
a gradient, else one launch per parameter with its group's ``lr`` and ``weight_decay``,
skipping parameters without a gradient as adam.py:97-104 does. Moments — and, for float16
models, float32 master weights (adam.py:75-81) — live on the device; ``m``, ``v`` and
``masters`` read them back in the reference's layouts. After a step the host Tensors are
stale until ``GPT.sync_to_host()`` (``save`` and ``save_checkpoint`` call it).

The parameters must belong to one ``nimbleml_amd.GPT`` (any subset of
``model.parameters()``).
"""
from __future__ import annotations

import numpy as np

from nimbleml_amd import _native as N


def _owner(params):
    from nimbleml_amd.gpt import _MODELS

    ids = {id(p) for p in params}
    for model in list(_MODELS):
        if ids <= {id(p) for p in model.parameters()}:
            return model
    raise TypeError("the device optimizer takes parameters of one nimbleml_amd.GPT "
                    "(e.g. model.parameters())")


class Adam:
    """Adam (no weight decay unless a parameter group sets one); adam.py:44-88."""

    def __init__(self, params, learning_rate=0.001, beta1=0.9, beta2=0.999, epsilon=1e-8, *,
                 lr=None):
        params = list(params)
        default_lr = lr if lr is not None else learning_rate
        if params and isinstance(params[0], dict):  # optimizer.py:17-27
            self.param_groups = []
            for group in params:
                if "params" not in group:
                    raise ValueError("each param group must include 'params'")
                entry = {"params": list(group["params"]),
                         "lr": group.get("lr", group.get("learning_rate", default_lr))}
                if "weight_decay" in group:
                    entry["weight_decay"] = float(group["weight_decay"])
                self.param_groups.append(entry)
        else:
            self.param_groups = [{"params": params, "lr": default_lr}]
        self.params = [p for g in self.param_groups for p in g["params"]]
        self.model = _owner(self.params)
        # fp16 compute: gradients accumulate in float32 (optimizer.py:33-38)
        if self.model._dtype == np.float16:
            for p in self.params:
                p._grad_dtype = np.float32
        self.beta1 = beta1
        self.beta2 = beta2
        self.epsilon = epsilon
        self.weight_decay = 0.0
        self._state_dtype = np.float32
        self.t = 0

    # ------------------------------------------------------- optimizer.py:44-100
    @property
    def learning_rate(self):
        return self.param_groups[0]["lr"]

    @learning_rate.setter
    def learning_rate(self, value):
        for group in self.param_groups:
            group["lr"] = value

    def get_lr(self):
        return [group["lr"] for group in self.param_groups]

    def set_lr(self, lrs):
        if len(lrs) != len(self.param_groups):
            raise ValueError(f"expected {len(self.param_groups)} learning rates, got {len(lrs)}")
        for group, value in zip(self.param_groups, lrs):
            group["lr"] = value

    def zero_grad(self, set_to_none: bool = False):
        for p in self.params:
            p.zero_grad(set_to_none=set_to_none)

    # ------------------------------------------------------------------- step
    def step(self):
        """adam.py:85-128 on the device."""
        self.t += 1
        bc1 = 1.0 - self.beta1 ** self.t
        bc2 = 1.0 - self.beta2 ** self.t
        live = [p for p in self.params if p.grad is not None]
        if not live:
            return
        model = self.model
        h = model._adam_state_ready()
        model._push_grads(live)
        args = (float(self.beta1), float(self.beta2), float(bc1), float(bc2), float(self.epsilon))
        everything = {id(p) for p in model.parameters()}
        if len(self.param_groups) == 1 and len(live) == len(everything) and \
                {id(p) for p in live} == everything:
            g = self.param_groups[0]
            wd = float(g.get("weight_decay", self.weight_decay))
            N.check(N.lib.nml_model_adamw_step(h, float(g["lr"]), *args, wd))
        else:
            ranges = model._param_ranges()
            for g in self.param_groups:
                wd = float(g.get("weight_decay", self.weight_decay))
                for p in g["params"]:
                    if p.grad is None:
                        continue
                    kind, layer, off, n = ranges[id(p)]
                    N.check(N.lib.nml_model_adamw_update(h, kind, layer, off, n, float(g["lr"]),
                                                         *args, wd))
        N.check(N.lib.nml_synchronize())
        model._host_stale = True

    # ------------------------------------------------------------------ state
    def _state(self, which):
        model = self.model
        model._adam_state_ready()
        vals = model._adam_read(which, self.params)
        return [vals[id(p)].reshape(-1) for p in self.params]

    @property
    def m(self):
        """First moments, one flat float32 array per parameter (adam.py:72)."""
        return self._state("m")

    @property
    def v(self):
        """Second moments, one flat float32 array per parameter (adam.py:73)."""
        return self._state("v")

    @property
    def masters(self):
        """float32 master weights of a float16 model, else None per parameter (adam.py:75-81)."""
        if self.model._dtype != np.float16:
            return [None] * len(self.params)
        return self._state("master")

    def _load_state(self, m, v, masters=None):
        """Write moments (and masters) given per parameter in the reference's layouts."""
        model = self.model
        model._adam_state_ready()
        model._adam_write("m", {id(p): a for p, a in zip(self.params, m)})
        model._adam_write("v", {id(p): a for p, a in zip(self.params, v)})
        if masters is not None and model._dtype == np.float16:
            model._adam_write("master", {id(p): a for p, a in zip(self.params, masters)
                                         if a is not None})


class AdamW(Adam):
    """Adam with decoupled weight decay (adam.py:293-311)."""

    def __init__(self, params, learning_rate=0.001, beta1=0.9, beta2=0.999, epsilon=1e-8,
                 weight_decay=0.01, *, lr=None):
        super().__init__(params, learning_rate=learning_rate, beta1=beta1, beta2=beta2,
                         epsilon=epsilon, lr=lr)
        self.weight_decay = float(weight_decay)
