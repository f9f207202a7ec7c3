"""spiky_amd: MI355X-native (gfx950) LUT-layer hot path with the reference
Spiky LUT API (LUTForwardFN, LUTLayer, ProjectionLUTLayer, LUTTransformer)."""
from . import _native  # noqa: F401
from .lut.lut_data_manager import LUTDataManagerF, LUTDataManagerI  # noqa: F401
from .lut.LUTTransformer import LUTTransformer  # noqa: F401
from .lut.LUTLayer import (  # noqa: F401
    GradientPolicy, GradientType, LUTLayer, LUTLayerBasic, LUTSharedContext, Conv2DLUTLayer,
    ProjectionLUTLayer, SynapseMeta,
)

__version__ = "0.1.0"
