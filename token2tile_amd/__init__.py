"""Token2Tile sparse attention, MI355X-native (gfx950 HIP kernels behind a C ABI).

``operator_dir()`` returns the directory of the operator module
(``deploy_step.py``) like ``token2tile.operator_dir()``.
"""
from pathlib import Path

__version__ = "0.1.0"


def operator_dir() -> str:
    """Directory of the attention operator (deploy_step.py and the HIP library)."""
    return str(Path(__file__).resolve().parent)
