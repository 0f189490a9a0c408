"""gsx_amd - an MI355X (gfx950) backend for the gsx 3D Gaussian Splatting library.

The compute lives in libgsx_hip.so (hand-written HIP kernels behind the C ABI declared in
include/gsx_hip.h). This package holds the ctypes binding (_lib), a host-side mirror of gsx's
renderer / loss / optimizer interface (backend) and the seeded benchmark scenes (scenes).
"""
import os

HERE = os.path.dirname(os.path.abspath(__file__))
