"""Import name for the package directory ``metal-gauss_amd/``.

A hyphen is not valid in a Python module name, so this module loads that
directory as the package ``metal_gauss_amd`` and replaces itself with it in
``sys.modules``; ``import metal_gauss_amd.backend`` and friends then resolve
inside the directory as usual.
"""

import importlib.util
import sys
from pathlib import Path

_DIR = Path(__file__).resolve().parent / "metal-gauss_amd"
_spec = importlib.util.spec_from_file_location(
    __name__, _DIR / "__init__.py", submodule_search_locations=[str(_DIR)])
_pkg = importlib.util.module_from_spec(_spec)
sys.modules[__name__] = _pkg
_spec.loader.exec_module(_pkg)
