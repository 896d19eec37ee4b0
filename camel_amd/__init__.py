"""camel_amd -- MI355X (gfx950) backend of the Camel `tensor` module hot path.

Native parts (built in-tree by ``python -m camel_amd.build``):
  lib/libcamel_hip.so     HIP kernels behind the C-ABI of include/camel_hip.h
  lib/libcamel_tensor.so  C++ operator layer: the tensor:* operators and the
                          device-resident TensorObject (include/camel_tensor.h)
Python: ``_hip`` (ctypes binding of the C-ABI), ``datagen`` (seeded inputs).
"""
__all__ = ["_hip", "datagen"]
