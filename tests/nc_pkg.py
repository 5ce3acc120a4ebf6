"""Imports the product package from its directory (its name contains a dot)."""
import importlib.util
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "nanochatllms.cpp_amd")


def _load():
    if "nanochat_amd" in sys.modules:
        return sys.modules["nanochat_amd"]
    spec = importlib.util.spec_from_file_location("nanochat_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["nanochat_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


nc = _load()
