"""MI355X-native replacement for QVGGT's ``awq_inference_engine`` hot path.

* ``qvggt_amd.awq_inference_engine`` -- the 14 ops of the reference extension
  (same names and signatures), backed by libqvggt_hip.so.
* ``qvggt_amd.awq.WQLinear`` -- the quantised linear module (same buffers).
"""
__version__ = "0.1.0"
