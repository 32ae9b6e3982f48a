"""Support modules: error types and environment options."""
