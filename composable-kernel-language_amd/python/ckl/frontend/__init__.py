from .emitter import LoweredProgram
from .source import INTRINSICS, FrontendError, block, kernel, program

__all__ = ["FrontendError", "LoweredProgram", "block", "kernel", "program"]
