"""Registers torch.ops.st.* (counterpart of silvertorch/ops/_load_ops.py:29-42).

Imports the in-tree extension ``silvertorch_amd._C``, whose static
initialisers register the operators.  There is no fallback: a missing or
unloadable extension raises ImportError.
"""

import importlib

import torch  # noqa: F401  (loads libtorch before the extension)

try:
    importlib.import_module("silvertorch_amd._C")
except ImportError as _e:
    raise ImportError(
        "silvertorch_amd HIP extension not found or not loadable; build it with "
        "`python -m silvertorch_amd._build` (there is no CPU fallback)"
    ) from _e
