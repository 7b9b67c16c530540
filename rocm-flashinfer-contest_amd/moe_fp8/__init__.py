"""MI355X (gfx950) fp8 block-scale MoE operator behind the reference's ``run(...)`` API."""
from .main import BLOCK, E_GLOBAL, H, I, N_GROUP, TOP_K, TOPK_GROUP, quantize_hidden, route, run  # noqa: F401
