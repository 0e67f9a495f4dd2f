"""KV connector formats: the identity profile, the ``tqp-kv-npz/1`` record
codec and the block store (turboquant_pro/connectors/), with the gfx950
plugins behind ``save``/``load``."""

from .identity import IncompatibleProfile, KVIdentityProfile, prefix_block_hashes  # noqa: F401
from .records import BLOB_CODEC, BlockRecord, rec_from_blob, rec_to_blob  # noqa: F401
from .store import ENCODER_VERSION, STATE_SCHEMA, TurboQuantBlockStore  # noqa: F401
from .vllm import TurboQuantKVConnector  # noqa: F401
