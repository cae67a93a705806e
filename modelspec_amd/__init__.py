"""modelspec-hip: an MI355X (gfx950) execution backend for ModelSpec training steps.

The product is libmsx.so (C ABI in include/msx.h). This package loads it and mirrors the
reference host's `train --backend hip` entry points (crates/modelspec-cli/src/train.rs).
"""
from .api import (  # noqa: F401
    CONFIGS,
    Context,
    MsxError,
    compile_config,
    device_count,
    lib,
)
