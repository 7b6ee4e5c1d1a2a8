"""The paged KV token write under the reference's module path.

``tensorforge/kernels/triton_cache.py`` is where the reference's decode
bucket imports ``paged_kv_write_token`` from
(``runtime/decode_bucket.py:21``).  This module exposes the gfx950
implementation (``tensorforge_amd.kernels.cache_write``) under the same
name, so a caller changes only the package prefix.
"""

from __future__ import annotations

from tensorforge_amd.kernels.cache_write import paged_kv_write_token

__all__ = ["paged_kv_write_token"]
