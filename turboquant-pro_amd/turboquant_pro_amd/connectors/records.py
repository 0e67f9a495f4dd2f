"""The KV block record and its blob codec, ``tqp-kv-npz/1``.

A record is one saved layer block: the key and value containers of the two
plugins plus the geometry needed to restore it (turboquant_pro/connectors/
vllm_v1.py:200-210).  Its blob is the reference's interchange framing
(vllm_v1.py:66-198), kept byte for byte so that stores written here and by
the reference read each other's records:

* an ``np.savez`` archive (no pickle anywhere) whose first member,
  ``__header__``, is the UTF-8 JSON header as a uint8 array, followed by
  ``k.<field>`` then ``v.<field>`` for every array field of the key and
  value containers, in the containers' field order;
* the header: ``codec``, ``shape``, ``dtype``, ``num_tokens``, ``head_dim``,
  ``n_heads``, then ``key_scalars`` / ``value_scalars`` holding every
  non-array field in field order (``None`` as null, dtypes as
  ``{"__dtype__": name}``, tuples as ``{"__tuple__": [...]}``).

Decoding refuses other codec versions, blobs or decompressed arrays beyond
``max_bytes``, and dtypes outside a numeric whitelist.
"""

from __future__ import annotations

import dataclasses
import io
import json
import types
from typing import Any

import numpy as np

__all__ = ["BLOB_CODEC", "BlockRecord", "RawTokens", "payload_to_state", "payload_from_state",
           "rec_to_blob", "rec_from_blob", "payload_nbytes"]

BLOB_CODEC = "tqp-kv-npz/1"
_NUMERIC_DTYPES = frozenset(("uint8", "int8", "int16", "int32", "int64", "float16", "float32",
                             "float64", "bool"))


@dataclasses.dataclass
class BlockRecord:
    """One saved layer block (vllm_v1.py:200-210)."""

    key_payload: Any
    value_payload: Any
    shape: tuple
    dtype: str
    num_tokens: int
    head_dim: int
    n_heads: int


@dataclasses.dataclass
class RawTokens:
    """Tokens kept as they are, fp16 or fp32 ``(1, H, n, D)`` (the pool's
    precision): the payload of the hot window's records in a pool's live-path
    save (``<layer>#hot<i>``), so a restore gives back exactly what the pool
    held.  A format of this library only.  Its blob member is
    ``k.data`` / ``v.data``; a reader without this payload type sees a record
    its quantizer cannot decode, which the store treats as a miss."""

    data: np.ndarray


def payload_nbytes(payload: Any) -> int:
    """Bytes held in the container's arrays."""
    return int(sum(v.nbytes for v in vars(payload).values() if isinstance(v, np.ndarray)))


def _scalar_state(name: str, value: Any) -> Any:
    if isinstance(value, np.dtype) or type(value).__name__.endswith("DType"):
        return {"__dtype__": str(np.dtype(value))}
    if isinstance(value, tuple):
        return {"__tuple__": list(value)}
    if value is None or isinstance(value, (bool, int, float, str)):
        return value
    raise TypeError(f"container field {name} of type {type(value).__name__} has no blob form")


def payload_to_state(payload: Any) -> tuple[dict, dict]:
    """Split a container into (array fields, JSON scalar fields), both in the
    container's field order (vllm_v1.py:76-99)."""
    arrays, scalars = {}, {}
    for name, value in vars(payload).items():
        if isinstance(value, np.ndarray):
            arrays[name] = value
        else:
            scalars[name] = _scalar_state(name, value)
    return arrays, scalars


def payload_from_state(arrays: dict, scalars: dict, cls: type | None = None) -> Any:
    """Rebuild a container: a namespace with the arrays then the scalars
    (vllm_v1.py:102-115), or an instance of the dataclass ``cls`` when given
    (every one of its fields must be present)."""
    values = dict(arrays)
    for name, value in scalars.items():
        if isinstance(value, dict) and "__dtype__" in value:
            value = np.dtype(value["__dtype__"])
        elif isinstance(value, dict) and "__tuple__" in value:
            value = tuple(value["__tuple__"])
        values[name] = value
    if cls is None:
        return types.SimpleNamespace(**values)
    names = [f.name for f in dataclasses.fields(cls)]
    missing = [n for n in names if n not in values]
    extra = [n for n in values if n not in names]
    if missing or extra:
        raise ValueError(f"record fields do not match {cls.__name__}: missing {missing}, extra {extra}")
    return cls(**values)


def rec_to_blob(rec: BlockRecord) -> bytes:
    """One record as one blob (vllm_v1.py:118-143)."""
    k_arrays, k_scalars = payload_to_state(rec.key_payload)
    v_arrays, v_scalars = payload_to_state(rec.value_payload)
    header = {"codec": BLOB_CODEC, "shape": list(rec.shape), "dtype": rec.dtype,
              "num_tokens": rec.num_tokens, "head_dim": rec.head_dim, "n_heads": rec.n_heads,
              "key_scalars": k_scalars, "value_scalars": v_scalars}
    members = {"__header__": np.frombuffer(json.dumps(header).encode(), dtype=np.uint8)}
    members.update((f"k.{n}", a) for n, a in k_arrays.items())
    members.update((f"v.{n}", a) for n, a in v_arrays.items())
    out = io.BytesIO()
    np.savez(out, **members)
    return out.getvalue()


def rec_from_blob(blob: bytes, max_bytes: int = 1 << 30, key_cls: type | None = None,
                  value_cls: type | None = None) -> BlockRecord:
    """Decode one blob (vllm_v1.py:146-195), refusing what it cannot vouch for."""
    if len(blob) > max_bytes:
        raise ValueError(f"blob exceeds max_bytes ({len(blob)} > {max_bytes})")
    k_arrays, v_arrays = {}, {}
    with np.load(io.BytesIO(blob), allow_pickle=False) as z:
        header = json.loads(bytes(z["__header__"]).decode())
        if header.get("codec") != BLOB_CODEC:
            raise ValueError(f"unknown record codec {header.get('codec')!r}; this reader handles "
                             f"{BLOB_CODEC!r} only (refusing, not guessing)")
        total = 0
        for name in z.files:
            if name == "__header__":
                continue
            arr = z[name]
            if str(arr.dtype) not in _NUMERIC_DTYPES:
                raise ValueError(f"dtype {arr.dtype} of {name} is not a whitelisted numeric dtype")
            total += arr.nbytes
            if total > max_bytes:
                raise ValueError("decompressed size exceeds max_bytes")
            if name.startswith("k."):
                k_arrays[name[2:]] = arr
            elif name.startswith("v."):
                v_arrays[name[2:]] = arr
    return BlockRecord(
        key_payload=payload_from_state(k_arrays, header["key_scalars"], key_cls),
        value_payload=payload_from_state(v_arrays, header["value_scalars"], value_cls),
        shape=tuple(header["shape"]), dtype=header["dtype"], num_tokens=int(header["num_tokens"]),
        head_dim=int(header["head_dim"]), n_heads=int(header["n_heads"]))
