"""tierlm_amd - MI355X (gfx950) HIP tier for tierlm's quantised-MoE decode path.

The compute lives in ``libtlm_hip.so`` (hand-written HIP, C ABI in
include/tlm_hip.h); this package only binds it.  There is no CPU fallback:
importing fails if the library is not built.
"""
from ._lib import EXPORTS, LIB_PATH, HipError, lib  # noqa: F401
from . import quant  # noqa: F401
from .moe import MoeBlock, MoeStack  # noqa: F401
