"""yaxus_amd: yaxus's paged KV-cache path on MI355X (gfx950).

- ``yaxus_amd.kv``       KvCache: page pool, prefix reuse, fork / copy-on-write, PassMeta
- ``yaxus_amd.backend``  HipBackend: arena, page copies, pass metadata, append, attention
- ``yaxus_amd.model``    the forward-pass order of the path (append -> copies -> layers)
- ``yaxus_amd.data``     the configurations' seeded synthetic inputs
"""

from .kv import KvCache, KvError, PageCopy, PassMeta, PassRows, SeqId  # noqa: F401
