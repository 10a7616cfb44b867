"""Every module of the package imports on a host without a GPU (no device work at import time)."""
import importlib
import pkgutil

import lockstep_amd


def test_every_module_imports():
    names = [m.name for m in pkgutil.iter_modules(lockstep_amd.__path__, "lockstep_amd.")
             if not m.name.split(".")[-1].startswith("lib")]   # (the shared library itself)
    assert names
    for name in names:
        importlib.import_module(name)
