"""atlas_amd -- MI355X (gfx950) implementation of ATLAS's single-token decode hot path.

Hand-written HIP kernels behind a C ABI (include/atlas_kernels.h,
include/atlas_engine.h), with host mirrors of the reference's Rust surface:
`tensor` (atlas-tensor), `quant` (atlas-quant), `model` (atlas-model decode),
`infer` (atlas-infer).  Build the library with `python -m atlas_amd.build`.
"""
from ._lib import AtlasError, LIB_PATH, load  # noqa: F401

__all__ = ["AtlasError", "LIB_PATH", "load"]
