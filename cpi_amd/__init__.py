"""cpi_amd — MI355X-native (gfx950) batch-1 decode engine for CPI-format
(.ll2c) Llama-family models.  The compute path is libcpi_hip.so (hand-written
HIP kernels behind the C-ABI in include/cpi_hip.h) driven by the C++ engine in
libcpi_engine.so; Python here is packaging and test plumbing."""

__version__ = "0.1.0"
