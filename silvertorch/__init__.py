"""The reference package's import path over this build.

Callers written against the reference import ``silvertorch.ops._load_ops``
(silvertorch/ops/_load_ops.py:29-42) and ``silvertorch.modules``
(silvertorch/modules/__init__.py); these modules resolve those paths to
``silvertorch_amd``, so such code runs unchanged.  Nothing here adds
behaviour: every name is the ``silvertorch_amd`` object itself.
"""

from silvertorch_amd import __version__  # noqa: F401
