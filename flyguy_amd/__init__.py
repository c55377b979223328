"""flyguy_amd: the fly actor's batched inference and sparse-hop trainer on one AMD MI355X.

A drop-in for the reference's flyguy fly actor path: FlyActor (flyguy_amd.fly), NativeFlyActor / NativeAdam /
grad_arrays (flyguy_amd.fly_native), the HopCuda-style hop (flyguy_amd.fly_hip), the NET.bin / PARAMS.bin formats
(flyguy_amd.export), over the C-ABI library flyguy_amd/libflyguy_core.so (include/flyguy_core.h).
"""
from .fly import FlyActor  # noqa: F401
