"""Stage B: sparse paged attention over the selected pages."""
from .decode import (ResidentVSource, decode_dense, decode_merge, decode_splitk, decode_splitk_tier,  # noqa: F401
                     ensure_stage_b_buffers, sparse_paged_decode_batched)
from .mla_decode import mla_decode, mla_decode_dense  # noqa: F401
