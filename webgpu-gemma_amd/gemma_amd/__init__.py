"""Python mirror of the MI355X Gemma-3 Q8_0 token loop's C-ABI (libgg.so).

Used by the tests, the benchmark and __graft_entry__; the product host for
applications is the JS engine in ../host, which calls the same C-ABI.
"""
from . import capi, gguf, synth  # noqa: F401
