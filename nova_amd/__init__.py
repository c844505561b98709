"""nova_amd — the int8 KV-cache decode path of Nova, built for MI355X (gfx950).

Modules mirror the reference's (captain-wangrun-cn/Nova, ``src/nova``):

- ``nova_amd.kvquant``  int8 quantize / dequantize (``nova.kvquant``'s int8 path)
- ``nova_amd.kvattn``   ``int8_attn_decode``, ``pack_int8_kv``, ``tail_attend``, ``KVInt8Cache``
- ``nova_amd.decode``   ``GraphDecoder(quant="int8")``, ``bucket_for``
- ``nova_amd.cache``    ``StaticKVCache`` (fp16 prefill staging)
- ``nova_amd.kernels``  ``hip_available()`` gate
- ``nova_amd.skeleton`` a random-weight attention-only decoder that drives the path

All compute runs in the HIP kernels of ``nova_amd/libnova_kv.so`` (C ABI in
``include/nova_kv.h``); build it with ``python -m nova_amd.build``.
"""

__all__ = ["kvquant", "kvattn", "decode", "cache", "kernels", "skeleton"]
