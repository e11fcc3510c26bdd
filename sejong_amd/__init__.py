"""sejong_amd -- MI355X (gfx950) native training step for Sejong's byte
Transformer: hand-written HIP kernels behind a C ABI (include/sejong_hip.h,
libsejong_hip.so) plus the host-side mirror of the reference's model /
optimizer interface."""
from . import _native  # noqa: F401  (raises ImportError if the library is not built)
from .model import Model, ModelConfig, TrainConfig, config, init_params, layout, byte_batch  # noqa: F401
