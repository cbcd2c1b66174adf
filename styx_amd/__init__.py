"""styx_amd: MI355X (gfx950) implementation of the styx / moe-stream MoE
decode hot path.  The compute lives in libstyx_hip.so (hand-written HIP for
gfx950, C ABI in include/styx_hip.h); this package is the Python mirror of
the reference's backend and engine interfaces over that library."""
from ._lib import (F16, F32, Q4_K, Q5_K, Q6_K, Q8_0, SKIP, StyxError, load)  # noqa: F401
from .model import (CFG_30B_A3B, CFG_LAYER_Q8, Hud, MoeModel, SynthConfig, argmax_last,  # noqa: F401
                    generate_hud)
from .runtime import Batch, Buffer, Gpu, Kernel  # noqa: F401
