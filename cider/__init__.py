"""cider - the reference package's import path, served by ``cider_amd``.

Code written against the reference imports ``cider`` (``cider/__init__.py:18-57``
of the reference): ``from cider import convert_model``,
``from cider.nn import CiderLinear``, ``from cider.ops import perchannel_linear``,
``import cider.convert``.  This package makes those imports resolve to the
MI355X implementation: ``cider.ops``, ``cider.nn`` and ``cider.convert`` are
the very module objects ``cider_amd.ops``, ``cider_amd.nn`` and
``cider_amd.convert`` (registered under both names), and the top-level names
are ``cider_amd``'s public surface.

One difference from the reference is deliberate: the reference replaces its
entry points by no-op stubs when the hardware is missing
(``cider/__init__.py:58-75``); here every entry point that needs the HIP
extension raises ``RuntimeError`` instead, and ``is_available()`` reports
whether it can run.
"""

import sys as _sys

import cider_amd as _impl
from cider_amd import convert as _convert
from cider_amd import nn as _nn
from cider_amd import ops as _ops
from cider_amd import *  # noqa: F401,F403  (the public surface)
from cider_amd import __all__  # noqa: F401

__version__ = _impl.__version__

for _name, _mod in (("ops", _ops), ("nn", _nn), ("convert", _convert)):
    _sys.modules[f"{__name__}.{_name}"] = _mod
    globals()[_name] = _mod
del _name, _mod
