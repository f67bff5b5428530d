"""Model patches that route attention through the gfx950 kernels."""

from .qwen3 import (DeviceMetadata, device_metadata, qwen3_cache_allocator, qwen3_model_loader,  # noqa: F401
                    qwen3_model_patcher)
