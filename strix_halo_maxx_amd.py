"""Import name for the package directory strix-halo-maxx_amd/ (a directory name Python cannot import directly).

`import strix_halo_maxx_amd` loads strix-halo-maxx_amd/__init__.py as the package `strix_halo_maxx_amd`, so its
submodules import as `strix_halo_maxx_amd.ops`, `strix_halo_maxx_amd.md2`, ...
"""
import importlib.util
import os
import sys

_dir = os.path.join(os.path.dirname(os.path.abspath(__file__)), "strix-halo-maxx_amd")
_spec = importlib.util.spec_from_file_location(__name__, os.path.join(_dir, "__init__.py"),
                                               submodule_search_locations=[_dir])
_mod = importlib.util.module_from_spec(_spec)
sys.modules[__name__] = _mod
_spec.loader.exec_module(_mod)
