"""accy_amd — an MI355X (gfx950) execution target for Accy tensor programs.

``accy_amd.tensor`` records programs with named axes and writes ACTP v1 wire bytes (the reference's
``tensor.define`` / ``Builder`` / ``Value`` / ``wire.encode``); ``accy_amd.hip`` runs them on one
MI355X through the C ABI in include/accy_hip.h (``run_hip`` is the drop-in for ``tensor.runCpu``).
"""
from . import tensor
from .tensor import Builder, Program, Spec, TensorError, Type, Value, define, spec

__all__ = ["tensor", "Builder", "Program", "Spec", "TensorError", "Type", "Value", "define", "spec",
           "run_hip", "Hip", "Session", "HipError"]


def __getattr__(name):
    # The HIP bindings load libaccy_hip.so lazily so that recording works on hosts without it.
    if name in ("run_hip", "Hip", "Session", "HipError"):
        import importlib
        return getattr(importlib.import_module(__name__ + ".hip"), name)
    raise AttributeError(name)
