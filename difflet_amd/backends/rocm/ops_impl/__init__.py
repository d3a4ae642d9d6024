"""The rocm backend's op implementations (one module per op family, as difflet.ops loads them)."""
