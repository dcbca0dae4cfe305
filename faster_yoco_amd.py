"""Import name of the package in faster-yoco_amd/, whose directory name is not a Python identifier: with the
repository root on sys.path, ``import faster_yoco_amd`` (or ``from faster_yoco_amd import zero1_fast``) loads that
package under this name.  Importing it loads the native libraries (built in-tree by __graft_entry__.build()) and
registers the PyTorch operators; a missing library raises RuntimeError."""
import importlib.util
import os
import sys

_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'faster-yoco_amd')
_spec = importlib.util.spec_from_file_location(__name__, os.path.join(_DIR, '__init__.py'),
                                               submodule_search_locations=[_DIR])
_pkg = importlib.util.module_from_spec(_spec)
sys.modules[__name__] = _pkg          # the import system returns what sys.modules holds once this file has run
try:
    _spec.loader.exec_module(_pkg)
except BaseException:
    sys.modules.pop(__name__, None)
    raise
