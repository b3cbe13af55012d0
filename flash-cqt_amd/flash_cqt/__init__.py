"""flash_cqt on MI355X: a drop-in for Flash-CQT's Python API whose fused
engine runs on hand-written HIP kernels for gfx950 (libflashcqt.so).

    from flash_cqt import OctCQT, SlicedCQT, Graphed
    from flash_cqt.fused import FusedOctCQT       # graph-replayable fast path
    from flash_cqt.trainable import TrainableCQT  # autograd through adjoint kernels

OctCQT is the pure-torch transform definition (any device); FusedOctCQT and
TrainableCQT require a GPU and the built HIP library and raise otherwise.
"""
from .oct_cqt import OctCQT
from .sliced import SlicedCQT
from .graphed import Graphed

__all__ = ["OctCQT", "SlicedCQT", "Graphed"]
