"""MI355X (gfx950) fast-matmul backend for inference ``F.linear``.

Importing the package root stays light (no torch, no GPU): it exposes the
certificate loader like the reference's root (``src/rdna3_fastmm/__init__.py``).
Plans live in ``rdna3_fastmm.runtime``, operators and the FX rewrite in
``rdna3_fastmm.linear``, the Dynamo backend in ``rdna3_fastmm.inductor``.
"""

from .certificate import ExpandedScheme, load_expanded_scheme

__version__ = "0.1.0"

__all__ = ["ExpandedScheme", "__version__", "load_expanded_scheme"]
