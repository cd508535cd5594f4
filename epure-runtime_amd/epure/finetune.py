"""Compressed-state fine-tuning: codebook and scales train, indices stay frozen.

Mirrors the reference API (epure/finetune.py:39-176).  One behavioural
difference: the fused HIP path is differentiable (its backward writes
grad_cb / grad_scale straight from the packed indices), so gradients reach
``cb`` and ``scale`` whichever path a forward takes.  The reference's
``trainable_forward`` set a flag that nothing read (finetune.py:135-143 vs
runtime.py:98-126); here the flag is honoured by ``PackedLinear`` and forces
the materialize path.
"""
import hashlib

import torch
import torch.nn as nn

from .runtime import PackedLinear, PackedWeight

MODES = ("scale", "codebook", "both")


def packed_weights(model):
    """Every packed store in the model with its owner's path (finetune.py:42-46)."""
    for name, mod in model.named_modules():
        if isinstance(mod, PackedLinear):
            yield name, mod.store


def make_trainable(model, mode="both", verbose=True):
    """Promote ``scale`` and/or ``cb`` buffers to fp32 Parameters (finetune.py:49-102)."""
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}")
    for p in model.parameters():
        p.requires_grad_(False)

    def promote(store, attr):
        cur = getattr(store, attr)
        if isinstance(cur, nn.Parameter):
            cur.requires_grad_(True)
            return cur
        store.__dict__.pop("_hot_cache", None)
        store.__dict__.pop("_hip_hot", None)
        store._buffers.pop(attr, None)
        setattr(store, attr, nn.Parameter(cur.detach().float().clone(), requires_grad=True))
        return getattr(store, attr)

    params, seen = [], set()
    for _, store in packed_weights(model):
        if id(store) in seen:
            continue
        seen.add(id(store))
        if mode in ("scale", "both"):
            params.append(promote(store, "scale"))
        if mode in ("codebook", "both"):
            params.append(promote(store, "cb"))
    if verbose:
        n_train = sum(p.numel() for p in params)
        print(f"  mode {mode}: {len(seen)} packed tensors, {n_train / 1e6:.2f}M trainable")
    return params


def snapshot_indices(model):
    """blake2b-128 of every store's packed bytes (finetune.py:105-117)."""
    return {name: hashlib.blake2b(store.packed.detach().cpu().numpy().tobytes(),
                                  digest_size=16).hexdigest()
            for name, store in packed_weights(model)}


def verify_frozen(model, snapshot):
    """Raise if any index buffer changed since ``snapshot`` (finetune.py:120-132)."""
    now = snapshot_indices(model)
    moved = [k for k, v in snapshot.items() if now.get(k) != v]
    if moved:
        raise RuntimeError(f"{len(moved)} index buffers changed during training "
                           f"(first: {moved[0]}). Indices must stay frozen.")
    return True


def trainable_forward(model, enable=True):
    """Force the materialize path for every packed linear (finetune.py:135-143)."""
    for _, store in packed_weights(model):
        store._force_materialize = enable
    return model


class ScaleTuner:
    """Minimal codebook/scale adaptation loop (finetune.py:146-176)."""

    def __init__(self, model, mode="both", lr=1e-4, device=None):
        self.model = model
        self.device = device or next((p.device for p in model.parameters()),
                                     torch.device("cpu"))
        self.params = make_trainable(model, mode)
        self.snapshot = snapshot_indices(model)
        self.opt = torch.optim.AdamW(self.params, lr=lr)

    def step(self, input_ids, labels=None):
        labels = input_ids if labels is None else labels
        out = self.model(input_ids.to(self.device), labels=labels.to(self.device))
        out.loss.backward()
        self.opt.step()
        self.opt.zero_grad(set_to_none=True)
        return float(out.loss.detach())

    def finish(self):
        verify_frozen(self.model, self.snapshot)
        for p in self.params:
            p.requires_grad_(False)
        return self.model


__all__ = ["MODES", "packed_weights", "make_trainable", "snapshot_indices", "verify_frozen",
           "trainable_forward", "ScaleTuner", "PackedWeight"]
