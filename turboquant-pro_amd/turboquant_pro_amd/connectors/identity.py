"""Identity of a persisted KV tier: the profile a stored block is valid under.

Same schema and digest as turboquant_pro/connectors/identity.py:45-238
(``tqp-kv-identity/1``): a store written by the reference and one written by
this build's GPU encode carry the same digest for the same configuration, so
blocks hand over between them.  The rules:

* every field takes part in the digest; ``None`` means unknown;
* a profile with an unknown field is incomplete and compatible with nothing,
  itself included (uncertain compatibility is a miss, never a best-effort
  decode);
* compatibility is digest equality of two complete profiles;
* the digest is SHA-256 over canonical JSON (sorted keys, compact separators,
  ASCII, non-finite floats refused) of the field dictionary;
* prefix hashes chain per whole block of token ids, seeded by the digest.
"""

from __future__ import annotations

import dataclasses
import hashlib
import json
from collections.abc import Sequence
from typing import Any

__all__ = ["KVIdentityProfile", "IncompatibleProfile", "prefix_block_hashes", "SCHEMA"]

SCHEMA = "tqp-kv-identity/1"


class IncompatibleProfile(Exception):
    """A profile gate refused: mismatch, incompleteness, or no profile."""


def canonical_json(obj: Any) -> str:
    """The digest's canonical text of ``obj`` (identity.py:48-56)."""
    return json.dumps(obj, sort_keys=True, separators=(",", ":"), ensure_ascii=True,
                      allow_nan=False)


def _sha256_hex(text: str) -> str:
    return hashlib.sha256(text.encode()).hexdigest()


@dataclasses.dataclass(frozen=True)
class KVIdentityProfile:
    """Configuration that can change a KV block's bytes (identity.py:59-103).

    Field names and meanings are the reference's: model state, positional and
    attention configuration, shape and placement, and the quantization
    discipline (``quant``: plugin names and every parameter) with the encoder
    version.  Dict fields are canonicalised recursively by the digest."""

    model_repo: str | None = None
    model_revision: str | None = None
    weight_fingerprint: str | None = None
    tokenizer_fingerprint: str | None = None
    architecture: str | None = None
    adapter_identity: str | None = None
    rope: dict | None = None
    attention_backend: str | None = None
    kv_layout_version: str | None = None
    sliding_window: int | None = None
    n_layers: int | None = None
    n_heads: int | None = None
    n_kv_heads: int | None = None
    head_dim: int | None = None
    tp_size: int | None = None
    pp_size: int | None = None
    kv_dtype: str | None = None
    block_size: int | None = None
    quant: dict | None = None
    encoder_version: str | None = None
    schema: str = SCHEMA

    def as_dict(self) -> dict:
        return dataclasses.asdict(self)

    @property
    def unknown_fields(self) -> tuple[str, ...]:
        return tuple(name for name, value in self.as_dict().items()
                     if value is None and name != "schema")

    @property
    def is_complete(self) -> bool:
        return len(self.unknown_fields) == 0

    def digest(self) -> str:
        """SHA-256 of the canonical field dictionary (unknowns as null; defined
        for incomplete profiles too, for diagnostics only)."""
        return _sha256_hex(canonical_json(self.as_dict()))

    def compatible(self, other: "KVIdentityProfile | None") -> bool:
        if other is None or not (self.is_complete and other.is_complete):
            return False
        return self.digest() == other.digest()

    def require_compatible(self, other: "KVIdentityProfile | None") -> None:
        """Raise :class:`IncompatibleProfile` naming why ``other`` is refused."""
        if self.compatible(other):
            return
        if other is None:
            raise IncompatibleProfile("no profile supplied")
        unknown = sorted(set(self.unknown_fields) | set(other.unknown_fields))
        if unknown:
            raise IncompatibleProfile(
                f"incomplete profile: unknown fields {unknown} -- an uncertain "
                "match is a miss, never a best-effort decode")
        mine, theirs = self.as_dict(), other.as_dict()
        raise IncompatibleProfile(
            f"profile mismatch in fields {[k for k in mine if mine[k] != theirs.get(k)]}")


def prefix_block_hashes(profile: KVIdentityProfile, token_ids: Sequence[int], *,
                        block_size: int = 16) -> list[str]:
    """Chained content hashes of the whole ``block_size``-token blocks of a
    prefix (identity.py:206-238): ``h0 = H(digest)``, ``h_i = H(h_{i-1} + ":" +
    canonical(block i))``.  A trailing partial block gets no hash."""
    if not profile.is_complete:
        raise IncompatibleProfile(
            "cannot mint cache keys under an incomplete profile "
            f"(unknown: {sorted(profile.unknown_fields)})")
    ids = [int(t) for t in token_ids]
    chain = _sha256_hex(profile.digest())
    hashes = []
    for start in range(0, len(ids) // block_size * block_size, block_size):
        chain = _sha256_hex(chain + ":" + canonical_json(ids[start:start + block_size]))
        hashes.append(chain)
    return hashes
