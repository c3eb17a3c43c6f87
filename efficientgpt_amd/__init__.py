"""MI355X (gfx950) batch-1 int8 decode path: HIP kernels behind a C ABI, drop-in Python surface.

  efficientgpt_amd.int8_linear       efficientgpt::int8_linear op, Int8Linear, quantize_model
  efficientgpt_amd.decode_attention  split-K GQA decode attention and its dispatch
The HIP library (libegpt_hip.so) is loaded lazily on first use.
"""

__version__ = '0.1.0'
