"""compressai_amd -- MI355X-native (gfx950, HIP) VQ2 decode hot path.

Hand-written HIP kernels behind the C ABI of ``include/vq2_amd.h``
(``libvq2_amd.so``), with Python entry points that keep the reference's
``vq2.kernels`` names and signatures:

* ``compressai_amd.kernels``  VQ GEMV (2/3/4 bpw), grouped per-expert GEMV,
  RHT, router top-k, top-1, dequant and index-decode entry points;
* ``compressai_amd.rot``      ``Rot`` / ``get_rot`` / ``FastRot`` on the RHT kernel;
* ``compressai_amd.runtime``  ``PackedLinear`` / ``PackedLMHead`` callers;
* ``compressai_amd.moe``      resident expert pool module and full MoE layer;
* ``compressai_amd.synth``    seeded synthetic workloads.
"""
__version__ = "0.1.0"
