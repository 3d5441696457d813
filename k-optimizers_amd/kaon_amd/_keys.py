"""The launch-cache key of a parameter group: which params have a gradient, and
the param and gradient storage, gradient dtype, contiguity and layout, read in
one native pass (``_kaon_key``, csrc/kaon_key.cpp, built by csrc/build_key.py)."""
from __future__ import annotations

import os
import sysconfig

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_kaon_key" + sysconfig.get_config_var("EXT_SUFFIX"))

_mod = None


def _load():
    global _mod
    if _mod is None:
        if not os.path.exists(PATH):
            raise RuntimeError(f"kaon_amd: host helper not built ({PATH}); run "
                               "python k-optimizers_amd/csrc/build_key.py or __graft_entry__.build()")
        from . import _kaon_key
        _mod = _kaon_key
    return _mod


def group_key(params: list) -> tuple[list, bytes]:
    """(the params whose .grad is set, in order; the key bytes of them and their grads)."""
    return _load().group_key(params)
