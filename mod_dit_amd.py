"""Import shim: `import mod_dit_amd` loads the package kept in the `mod-dit_amd/` directory.

Python cannot import a hyphenated directory name directly, so this module loads
`mod-dit_amd/__init__.py` as the package `mod_dit_amd` and replaces itself with it.
"""
import importlib.util as _ilu
import sys as _sys
from pathlib import Path as _Path

_pkg_dir = _Path(__file__).resolve().parent / "mod-dit_amd"
_spec = _ilu.spec_from_file_location(__name__, _pkg_dir / "__init__.py",
                                     submodule_search_locations=[str(_pkg_dir)])
_mod = _ilu.module_from_spec(_spec)
_sys.modules[__name__] = _mod
_spec.loader.exec_module(_mod)
