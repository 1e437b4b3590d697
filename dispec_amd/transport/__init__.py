"""KV transfer payload layout (the transport buffer the gather kernel fills)."""
