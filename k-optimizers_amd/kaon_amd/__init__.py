"""kaon_amd -- MI355X (gfx950) HIP implementation of K-Optimizers' fused optimizer step.

Drop-in classes with the reference ``kaon`` API (constructors, ``step()``,
``state_dict`` layout, ``momentum_dtype`` / ``bf16_method`` knobs):
``Adakaon``, ``Lion``, ``Nekaon``, ``AdaMuon``, ``AdaPNM``, ``KProdigy``, ``MSAM``.  Every step runs hand-written HIP kernels
from ``libkaon_amd.so`` (C ABI in ``include/kaon_amd.h``); importing this
package does not load the library, the first step does, and fails loudly if it
has not been built.
"""
from ._base import fourbit_block_size, load_state_dict_preserving_dtypes
from .adakaon import Adakaon
from .adamuon import AdaMuon
from .adapnm import AdaPNM
from .kprodigy import KProdigy
from .lion import Lion
from .msam import MSAM
from .nekaon import Nekaon

__version__ = "0.1.0"
__all__ = ["AdaMuon", "AdaPNM", "Adakaon", "KProdigy", "MSAM", "Lion", "Nekaon", "fourbit_block_size", "load_state_dict_preserving_dtypes"]
