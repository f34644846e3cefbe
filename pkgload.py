"""Import helper for the ``vllm-neuron_amd/`` package directory.

The directory name carries a hyphen, so it is registered under the importable
name ``vllm_neuron_amd`` (``import vllm_neuron_amd.functional`` then works).
"""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG_DIR = ROOT / "vllm-neuron_amd"
NAME = "vllm_neuron_amd"


def load():
    if NAME in sys.modules:
        return sys.modules[NAME]
    spec = importlib.util.spec_from_file_location(
        NAME, PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[NAME] = mod
    spec.loader.exec_module(mod)
    return mod
