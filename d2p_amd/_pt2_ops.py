"""torch.compile entry points (placeholder until the d2p_py custom ops land).

``_ops._wrap`` routes compile-time and FakeTensor calls here when a matching
name exists; otherwise the raw ``torch.ops.d2p`` operator (with its fake
kernel from ``_compile``) is used.
"""
