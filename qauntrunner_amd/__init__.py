"""qauntrunner_amd -- MI355X (gfx950) paged-KV attention for QuantRunner.

The product is the C-ABI library ``libqr_attn.so`` (include/qr_attn.h) built
from ``csrc/``; this package holds its ctypes binding and the host-side
mirror of the reference classes PagedKvCache, MlaLatentCache, ModelStore and
PrefetchPipeline.
"""
from ._lib import (
    DTYPE_BF16,
    DTYPE_F16,
    DTYPE_F32,
    LIB_PATH,
    PAGE_TOKENS,
    QrError,
    QrHipError,
    QrInvalidArgument,
    QrNotResident,
    QrOutOfMemory,
    QrOutOfRange,
    load,
)
from .caches import MlaLatentCache, PagedKvCache, dtype_code
from .store import DeviceTensor, ModelStore, ModelStoreBuilder, PrefetchPipeline, TensorView
from .weights import Weight, matvec_dev, matvec_group_dev, mla_q_absorb_dev, mla_wuv_dev

__all__ = [
    "DTYPE_BF16", "DTYPE_F16", "DTYPE_F32", "LIB_PATH", "PAGE_TOKENS",
    "QrError", "QrHipError", "QrInvalidArgument", "QrNotResident", "QrOutOfMemory", "QrOutOfRange",
    "load", "MlaLatentCache", "PagedKvCache", "dtype_code",
    "Weight", "matvec_dev", "matvec_group_dev", "mla_q_absorb_dev", "mla_wuv_dev",
    "DeviceTensor", "ModelStore", "ModelStoreBuilder", "PrefetchPipeline", "TensorView",
]
