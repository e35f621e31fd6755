"""MI355X-native CacheBridge online handoff path (map + paged install).

Public API (mirrors the reference's mapper / online primitives):

- ``PageMapper`` / ``HeadwiseMapper`` (``cachebridge_amd.mapper``)
- ``PagedKVPool``, ``pool_rows`` (``cachebridge_amd.pool``)
- ``pack_source_block``, ``map_write_block``, ``map_install_block``,
  ``install_unpublished``, ``SourceLease`` (``cachebridge_amd.online.blocks``)
- ``PipelinedSourceLease``, ``StagedHandoff`` (``cachebridge_amd.online.pipeline``)

All compute runs in ``libcachebridge_hip.so`` (HIP, gfx950); importing the
package does not load it, the first plan or copy does, and raises if it is
not built.
"""

__version__ = "0.1.0"

from .mapper import HeadwiseMapper, PageMapper  # noqa: E402,F401
from .pool import PagedKVPool, pool_rows  # noqa: E402,F401
