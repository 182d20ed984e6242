"""GGUF container and GGML block layouts."""
from .gguf import (FLOAT_TYPES, GGMLType, GGUFFile, GGUFWriter, TYPE_LAYOUT, TensorInfo,  # noqa: F401
                   nbytes_for, row_geometry, tensor_info)
