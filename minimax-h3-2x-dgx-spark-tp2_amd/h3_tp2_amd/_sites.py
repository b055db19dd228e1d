"""Shared machinery of the block-scoped hook protocols (the producer stash of ``fp8_quant_fuse``, the consumer stash of
``fp8_consumers``, the weight routing of ``fp8_hip``).

* ``SITE_LAYERS`` / ``site_layer``: where each site's linear layer hangs off a MiniMax H3 DiT block.
* ``tracing``: True while torch.compile traces (the hooks stay out of traced graphs).
* ``Notes``: log a message the first time its key is seen.
* ``same_bits``: two tuples of tensors equal bit for bit (shape, dtype and every byte).
* ``checked``: the once-per-signature verdict of a fused form against the stock form on a row sample, kept in a
  caller-owned book (``book["checked"]`` verdicts, ``book["disabled"]`` sites), so a site is decided once per process.
"""
from __future__ import annotations

import contextlib
import logging
from typing import Any, Callable, Iterable

import torch

SITE_LAYERS = {"qkv": ("attn", "qkv_proj"), "out": ("attn", "out_proj"), "fc1": ("mlp", "fc1"), "fc2": ("mlp", "fc2")}


def site_layer(block, site: str):  # noqa: ANN001,ANN201
    """The linear layer of ``site`` in ``block`` (None when the block has no such layer)."""
    owner, name = SITE_LAYERS[site]
    return getattr(getattr(block, owner, None), name, None)


def layer_refusal(site: str, layer, lora_types) -> str | None:  # noqa: ANN001
    """Why ``site``'s layer cannot carry a block-scoped stash or route (None: it can): it must exist, be the plain
    layer (not a LoRA wrapper) and hold its whole output (a sharded layer's collective would read the placeholder)."""
    if layer is None:
        return f"{site}: the block has no {'.'.join(SITE_LAYERS[site])}"
    if lora_types and isinstance(layer, lora_types):
        return f"{site}: the layer sits inside a LoRA wrapper"
    shards = getattr(layer, "tp_size", 1)
    if shards != 1:
        return f"{site}: the layer is split over {shards} ranks (tp_size != 1)"
    return None


@contextlib.contextmanager
def block_scope(tls, scope):  # noqa: ANN001
    """``scope`` is the thread's running block scope (``tls.ctx``) while the body runs; the enclosing block's scope
    comes back afterwards.  A normal exit closes the scope (``scope.close()``: whatever the block left waiting is made
    real for whoever holds it); an exception drops it (``scope.drop()``) and propagates."""
    outer = getattr(tls, "ctx", None)
    tls.ctx = scope
    try:
        yield scope
    except BaseException:
        tls.ctx = outer
        scope.drop()
        raise
    tls.ctx = outer
    scope.close()


def tracing() -> bool:
    is_compiling = getattr(getattr(torch, "compiler", None), "is_compiling", None)
    return bool(is_compiling and is_compiling())


class Notes:
    """Warnings that are worth saying once per process each (keyed)."""

    def __init__(self, logger: logging.Logger, prefix: str):
        self.logger, self.prefix, self.seen = logger, prefix, set()

    def once(self, key: str, msg: str, *args: Any) -> None:
        if key not in self.seen:
            self.seen.add(key)
            self.logger.warning(self.prefix + msg, *args)


def _raw(t: torch.Tensor) -> torch.Tensor:
    """The tensor's bytes as integers of its element size (bitwise comparison; NaN equals the same NaN)."""
    t = t.contiguous()
    return t.view({1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()])


def same_bits(xs: Iterable[torch.Tensor], ys: Iterable[torch.Tensor]) -> bool:
    xs, ys = tuple(xs), tuple(ys)
    return len(xs) == len(ys) and all(
        x.shape == y.shape and x.dtype == y.dtype and torch.equal(_raw(x), _raw(y)) for x, y in zip(xs, ys))


def checked(book: dict, stats: dict, notes: Notes, key: tuple, fused: Callable[[], tuple],
            stock: Callable[[], tuple], *, disable_site: bool = True) -> bool:
    """The verdict for ``key`` (its first element names the site): on the first call, ``fused()`` against ``stock()``
    bit for bit (an exception counts as a mismatch); later calls return the recorded verdict.  A failing verdict with
    ``disable_site`` adds the site to ``book["disabled"]``."""
    verdicts = book["checked"]
    if key in verdicts:
        return verdicts[key]
    try:
        ok = same_bits(fused(), stock())
    except Exception as exc:  # noqa: BLE001  (a fused form that cannot even run is a failed check)
        notes.logger.warning(notes.prefix + "the fused form of %s failed to run (%s: %s)", key, type(exc).__name__,
                             exc)
        ok = False
    verdicts[key] = ok
    stats["selfcheck_pass" if ok else "selfcheck_fail"] += 1
    if not ok:
        if disable_site:
            book["disabled"].add(key[0])
        notes.logger.warning(notes.prefix + "self-check %s is not bit-identical to the stock form; %s", key,
                             f"site {key[0]} disabled" if disable_site else "trying the next form")
    return ok


def parse_site_list(value: str | None, sites: tuple) -> tuple:
    """A site selection from an environment-style string: "1" / "all" / "on" / "true" = every site, empty / "0" /
    "off" / "false" = none, otherwise a comma list (kept in the order of ``sites``)."""
    text = (value or "").strip().lower()
    every, none = {"1", "all", "on", "true"}, {"", "0", "off", "false"}
    if text in every:
        return tuple(sites)
    if text in none:
        return ()
    chosen = {part.strip() for part in text.split(",")}
    return tuple(site for site in sites if site in chosen)
