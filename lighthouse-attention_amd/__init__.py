"""MI355X-native Lighthouse selection attention.

The directory name is not a Python identifier, so it is loaded under the
module name ``lighthouse_attention_amd`` (see ``load_package`` in
``__graft_entry__.py``).  Inside a torchtitan checkout the package's
``lighthouse_selection.py`` replaces ``torchtitan/models/llama3/model/lighthouse_selection.py``
together with ``_native.py`` and ``liblighthouse_hip.so``.
"""
from . import _native
from .lighthouse_selection import *  # noqa: F401,F403
from .lighthouse_selection import __all__ as _api
from . import block_ops, dense_attention, llama3  # noqa: E402  (model kernels, dense layers, Llama3)

__all__ = list(_api) + ["_native", "block_ops", "dense_attention", "llama3"]
