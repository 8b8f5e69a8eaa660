"""ferric_amd — MI355X (gfx950) implementation of Ferric's Qwen3 forward-pass hot path.

The compute lives in libferric_hip.so (hand-written HIP kernels behind the C
ABI of include/ferric_hip.h). This package is the host-side mirror of the
reference's batch-runner interface plus a caller-side page pool for tests.
Importing it loads the shared library and fails loudly if it is missing.
"""

from ._lib import FerricError, load
from .pool import PagePool
from .runner import (QWEN3_0_6B, QWEN3_8B, BatchOutput, PagedLimits, PreparedBatch, PreparedRow,
                     TpBatchRunner)

load()

__all__ = ["FerricError", "PagePool", "PagedLimits", "PreparedBatch", "PreparedRow", "BatchOutput",
           "TpBatchRunner", "QWEN3_8B", "QWEN3_0_6B", "load"]
