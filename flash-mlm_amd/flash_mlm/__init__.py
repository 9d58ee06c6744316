"""flash_mlm on MI355X: fused non-causal (MLM) attention over packed / padded
sequences with a layer-scoped cached context, backed by hand-written gfx950 HIP
kernels (libflash_mlm_hip.so, C ABI in include/flash_mlm_hip.h).

Public names follow the reference package (src/flash_mlm/__init__.py:59-68).  The
compute functions need tensors on a HIP device and the built library; they raise
otherwise (there is no CPU path and no alternative backend).
"""

from flash_mlm.host.cache import InferenceCache, PackingCache, PackMetadata
from flash_mlm.host.host import (
    flash_attn_mlm,
    flash_attn_mlm_compressed,
    flash_attn_mlm_precompressed,
)
from flash_mlm.host.host_utils import build_pack_metadata, unpack_from_kernel

__version__ = "0.1.0"

__all__ = [
    "PackMetadata",
    "PackingCache",
    "InferenceCache",
    "build_pack_metadata",
    "unpack_from_kernel",
    "flash_attn_mlm",
    "flash_attn_mlm_compressed",
    "flash_attn_mlm_precompressed",
]
