"""heimdall_amd — MI355X-native (gfx950, HIP) kernels for the Bifrost converted-layer core of ValeroisAI/Heimdall.

Modules mirror the reference's interface for this path:
  kernels.delta_rule / delta_rule_step / delta_rule_varlen   (Heimdall/heimdall/kernels.py:132-155)
  motor.delta_rule_gqa                                       (Heimdall/heimdall/motor.py:70-102)
The compute runs in ``libbifrost_hip.so`` (C ABI in include/bifrost.h), loaded through ctypes.
"""
__version__ = "0.1.0"
