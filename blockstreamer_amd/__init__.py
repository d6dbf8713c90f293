"""blockstreamer_amd: BlockStreamer's gpt-oss MoE expert path, MI355X-native.

``blockstreamer_amd.gptoss`` mirrors ``block_streamer.gptoss``; the kernels
live in ``libbsamd.so`` (built from ``csrc/`` by ``blockstreamer_amd.build``).
"""

__version__ = "0.1.0"
