"""MI355X-native MoE layer (router, dispatch, grouped q4 SwiGLU experts,
combine) behind the C ABI of include/qmoe.h; see qmoe.py for the binding."""
from .qmoe import *  # noqa: F401,F403
from .qmoe import (BF16, F32, RESIDUAL, TAGS, WORKLOADS, AttentionContext, DecoderStack, DeltaNetContext,
                   GatedResidualContext, MoeContext, QmoeError, Workload, lib, load_library,
                   synth_fill, version, SIGNATURES, LIB_PATH, decoder_layer_types)  # noqa: F401

# load libqmoe.so now: a missing library is an import error, never a fallback
lib()
