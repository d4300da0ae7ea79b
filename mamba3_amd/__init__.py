"""mamba3_amd — MI355X-native (gfx950 HIP) Mamba-3 chunked-SSD forward path.

Drop-in for the public API of `mamba3` (mamba3/__init__.py:5-19): `import mamba3_amd as
mamba3` gives the same eight names.
"""

__version__ = "0.1.0"

from .layer import KulaMamba, RMSNorm
from .block import KulaMambaBlock, KulaMambaLM, SwiGLU
from .ssd import chunked_ssd, SSDOutput
from .scan import ssd_scan

__all__ = [
    "KulaMamba",
    "KulaMambaBlock",
    "KulaMambaLM",
    "RMSNorm",
    "SwiGLU",
    "SSDOutput",
    "chunked_ssd",
    "ssd_scan",
]
