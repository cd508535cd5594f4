"""Compressed-state fine-tuning: the codebook and the group scales learn, the
indices never move.

Public surface of the reference's epure/finetune.py:39-176 (``MODES``,
``packed_weights``, ``make_trainable``, ``snapshot_indices``,
``verify_frozen``, ``trainable_forward``, ``ScaleTuner``).

The weight of a packed linear is ``cb[idx] * scale``: with ``idx`` frozen it
is smooth in ``cb`` and ``scale``, so training is plain backprop into those
two small tensors.  In this build both routes carry the gradient: the fused
gfx950 kernels have their own backward (grad_cb / grad_scale straight from
the packed indices, ``epure.kernels.cuda``), and the materialize route is
differentiable.  ``trainable_forward`` therefore is not needed for
correctness; it forces the materialize route, which ``PackedLinear``
honours (the reference set a flag nothing read, runtime.py:98-126).
"""
import hashlib

import torch
import torch.nn as nn

from .runtime import PackedEmbedding, PackedLinear, PackedWeight

MODES = ("scale", "codebook", "both")

# which store tensors each mode trains
_TRAINED = {"scale": ("scale",), "codebook": ("cb",), "both": ("scale", "cb")}

# per-store caches that hold tensor pointers and must not outlive a swap
_POINTER_CACHES = ("_hip_hot", "_hot_cache")


def packed_weights(model):
    """``(module path, store)`` for every packed linear and packed embedding
    (finetune.py:42-46).  A store shared by two modules (tied lm_head) is
    reported under both paths."""
    for path, mod in model.named_modules():
        if isinstance(mod, (PackedLinear, PackedEmbedding)):
            yield path, mod.store


def _unique_stores(model):
    found = {}
    for _, store in packed_weights(model):
        found.setdefault(id(store), store)
    return list(found.values())


def _trainable(store, attr):
    """``store.<attr>`` as an fp32 leaf Parameter with grad on.

    A buffer is swapped for a Parameter once (a tied store is reached twice:
    the second visit reuses it); the swap drops the store's pointer caches,
    which would otherwise keep feeding the kernels the old tensor.
    """
    cur = getattr(store, attr)
    if not isinstance(cur, nn.Parameter):
        for key in _POINTER_CACHES:
            store.__dict__.pop(key, None)
        del store._buffers[attr]
        cur = nn.Parameter(cur.detach().to(torch.float32).clone())
        store.register_parameter(attr, cur)
    cur.requires_grad_(True)
    return cur


def make_trainable(model, mode="both", verbose=True):
    """Freeze the model, then make ``scale`` and/or ``cb`` of every packed
    store a trainable fp32 Parameter (finetune.py:49-102).  Returns the
    Parameters, per store ``scale`` before ``cb``."""
    if mode not in MODES:
        raise ValueError(f"mode {mode!r} is not one of {MODES}")
    model.requires_grad_(False)
    stores = _unique_stores(model)
    params = [_trainable(s, attr) for s in stores for attr in _TRAINED[mode]]
    if verbose:
        n_train = sum(p.numel() for p in params)
        n_idx = sum(s.out_features * s.in_features for s in stores)
        share = 100.0 * n_train / max(n_train + n_idx, 1)
        print(f"  mode {mode}: {len(stores)} packed stores, {n_train / 1e6:.2f}M trainable "
              f"values ({share:.2f}% of the weight values; indices frozen)")
    return params


def _digest(t):
    raw = t.detach().to("cpu").contiguous().view(torch.uint8).numpy()
    return hashlib.blake2b(raw.tobytes(), digest_size=16).hexdigest()


def snapshot_indices(model):
    """``{path: blake2b-128 hex of the store's packed bytes}`` (the digest of
    finetune.py:105-117): a byte hash, so swapped indices change it."""
    return {path: _digest(store.packed) for path, store in packed_weights(model)}


def verify_frozen(model, snapshot):
    """True if no index buffer differs from ``snapshot``; otherwise raises
    ``RuntimeError`` naming the stores whose indices changed (a store that
    disappeared counts as changed)."""
    now = snapshot_indices(model)
    changed = sorted(p for p, d in snapshot.items() if now.get(p) != d)
    if changed:
        shown = ", ".join(changed[:4]) + (" ..." if len(changed) > 4 else "")
        raise RuntimeError(f"packed indices are no longer frozen: {len(changed)} store(s) "
                           f"differ from the snapshot ({shown})")
    return True


def trainable_forward(model, enable=True):
    """Route every packed linear through ``materialize`` (``enable``) or back
    to the fused kernels (finetune.py:135-143)."""
    for store in _unique_stores(model):
        if enable:
            store._force_materialize = True
        else:
            store.__dict__.pop("_force_materialize", None)
    return model


def _device_of(model):
    for t in model.parameters():
        return t.device
    for t in model.buffers():
        return t.device
    return torch.device("cpu")


class ScaleTuner:
    """A minimal codebook/scale adaptation loop (finetune.py:146-176): AdamW
    on the Parameters ``make_trainable`` returns, causal-LM loss from
    ``model(input_ids, labels=...)``, and ``finish()`` proves the indices
    never moved before freezing the Parameters again."""

    def __init__(self, model, mode="both", lr=1e-4, device=None):
        self.model = model
        self.device = torch.device(device) if device is not None else _device_of(model)
        self.params = make_trainable(model, mode)
        self.snapshot = snapshot_indices(model)
        self.opt = torch.optim.AdamW(self.params, lr=lr)

    def step(self, input_ids, labels=None):
        """One optimizer step; returns the loss before the update."""
        ids = input_ids.to(self.device)
        target = ids if labels is None else labels.to(self.device)
        loss = self.model(ids, labels=target).loss
        self.opt.zero_grad(set_to_none=True)
        loss.backward()
        self.opt.step()
        return loss.item()

    def finish(self):
        verify_frozen(self.model, self.snapshot)
        for p in self.params:
            p.requires_grad_(False)
        return self.model


__all__ = ["MODES", "packed_weights", "make_trainable", "snapshot_indices", "verify_frozen",
           "trainable_forward", "ScaleTuner", "PackedWeight"]
