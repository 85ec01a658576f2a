"""Loads the factory test module (tests/factory/nott_factory.cpp, built by
tests/factory/Makefile against the reference's headers), or None when it was
not built (no reference sources where the tree was built)."""
import importlib
import os
import sys

_BUILD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "factory", "_build")


def load():
    if not os.path.isdir(_BUILD):
        return None
    if _BUILD not in sys.path:
        sys.path.insert(0, _BUILD)
    try:
        from thot_amd import _abi
        _abi.load()
        return importlib.import_module("_nott_factory")
    except ImportError:
        return None
