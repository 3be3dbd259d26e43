"""Stage A: rki4 summaries, per-page scores and exact top-b page selection."""
from .rki4_state import Rki4State, record_bytes  # noqa: F401
from .ops import (derive_page_params, rki4_score_only, rki4_score_state,  # noqa: F401
                  rki4_select_only, topb_select)
from .mla_state import MlaState  # noqa: F401
from .mla_select import (mla_build_blocks, mla_derive, mla_score_only,  # noqa: F401
                         mla_select_only, mla_select_pages)
from .rki4_build import (rki4_build_blocks, rki4_build_bulk, rki4_build_delta,  # noqa: F401
                         rki4_build_refresh, rki4_build_tail, rki4_pack)
