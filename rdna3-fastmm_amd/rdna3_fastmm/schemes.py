"""The verified schemes the runtime executes, with their block conventions.

Block numbering used everywhere in this package (kernels, oracle, plans):

* A side: signal ``i`` of ``left`` is block ``(i // s, i % s)`` of the
  activation ``x[M, K]`` (row block, column block), each block
  ``Mb x Kb`` with ``Mb = ceil(M/s)``, ``Kb = ceil(K/s)``; rows or columns past
  ``M``/``K`` read as zero (reference ``runtime.py:75-77``, generated
  ``left_transform_kernel`` masks).
* B side: signal ``j`` of ``right`` is block ``(j // s, j % s)`` of
  ``B = W^T [K, N]`` (K block, N block). For a Linear weight ``W[N, K]`` that
  is ``W[(j % s)*Nb + n, (j // s)*Kb + k]``.
* Output: output ``c`` of ``output`` is block ``(c // s, c % s)`` of
  ``C[M, N]``.

Each scheme is loaded and verified exactly (Brent identity, operation counts,
SHA-256) on first use.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache
import hashlib
from pathlib import Path

from .certificate import load_reduced_scheme, lower_reduced_scheme
from .program import LinearProgram
from .slp import load_and_verify_slp_certificate

CERTIFICATE_ROOT = Path(__file__).resolve().parent / "certificates"


@dataclass(frozen=True)
class Scheme:
    name: str
    algorithm: str
    size: int
    rank: int
    left: LinearProgram
    right: LinearProgram
    output: LinearProgram
    certificate: Path
    certificate_sha256: str
    scheme_id: int

    @property
    def dimensions(self) -> tuple[int, int, int]:
        return (self.size, self.size, self.size)


@dataclass(frozen=True)
class _Entry:
    name: str
    algorithm: str
    directory: str
    kind: str
    sha256: str
    scheme_id: int


# scheme_id is the integer the C ABI uses to select a scheme (include/fastmm_amd.h).
# The SHA-256 pins are the certificates the reference binds (runtime.py:30-47).
_ENTRIES = {
    "rank7": _Entry(
        "rank7_2x2x2", "rank7-v1", "2x2x2_rank7_15add", "reduced",
        "b374fcc797ea014994453b7502625e24f70ca2f1dcf1bdbe74a716342bfefb1e", 0,
    ),
    "rank48": _Entry(
        "rank48_4x4x4", "rank48-accurate-v1", "4x4x4_rank48_accurate", "slp",
        "c7103a1165af22d4e1a417607e9618b0bbae1b69e0c48ed7fa2a5aba26a3bcb7", 1,
    ),
    "rank49": _Entry(
        "rank49_4x4x4", "rank49-v1", "4x4x4_rank49_159add", "reduced",
        "a3c4121dfd09607045255628dd94b60133c24c46b65f1089e89c6564ba522561", 2,
    ),
    "rank343": _Entry(
        "rank343_8x8x8", "rank343-mfma-v1", "8x8x8_rank343_1661add", "reduced",
        "c7afccb09f8491e484af1696c25c809757c4af649ee7220e79f25d1c7afe3955", 3,
    ),
}

SCHEME_KEYS = tuple(_ENTRIES)


@lru_cache(maxsize=None)
def load_scheme(key: str) -> Scheme:
    entry = _ENTRIES[key]
    manifest = CERTIFICATE_ROOT / entry.directory / "certificate.json"
    if entry.kind == "reduced":
        circuit = lower_reduced_scheme(load_reduced_scheme(manifest))
        dimensions, rank = circuit.dimensions, circuit.rank
        left, right, output = circuit.left, circuit.right, circuit.output
        digest = hashlib.sha256(manifest.read_bytes()).hexdigest()
    else:
        certificate, summary = load_and_verify_slp_certificate(manifest)
        dimensions, rank = summary.dimensions, summary.rank
        left, right, output = certificate.left, certificate.right, certificate.output
        digest = summary.sha256
    if digest != entry.sha256:
        raise RuntimeError(f"{entry.name} certificate does not match its pinned SHA-256")
    if len(set(dimensions)) != 1:
        raise RuntimeError("only square block schemes are supported")
    return Scheme(
        name=entry.name,
        algorithm=entry.algorithm,
        size=dimensions[0],
        rank=rank,
        left=left,
        right=right,
        output=output,
        certificate=manifest,
        certificate_sha256=digest,
        scheme_id=entry.scheme_id,
    )
