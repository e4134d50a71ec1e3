from .emitter import LoweredProgram
from .source import FrontendError, INTRINSICS, kernel, program

__all__ = ["FrontendError", "LoweredProgram", "kernel", "program"]
