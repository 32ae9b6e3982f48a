"""Compiler-side modules of the backend: targets, the native call path and the
output pool."""
