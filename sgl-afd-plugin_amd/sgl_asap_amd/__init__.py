"""MI355X-native F-side routed-expert path of an attention-FFN disaggregated MoE plugin.

Host code mirrors the reference plugin's interfaces (``python/sgl_asap_plugin``): the
transport layout and channel (``transport/``), the A-side ``AsapMoE`` / ``AsapDispatcher``
surface and the F-side expert runner (``moe/``), the FFN scheduler's job handler and the
HIP-graph bucket runner (``runner/``). All arithmetic runs in hand-written gfx950 HIP
kernels in ``libafd.so`` (built from ``../csrc``), bound with ctypes (``_lib``).
"""

__version__ = "0.1.0"
