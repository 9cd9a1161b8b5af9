"""Engine-side integration of the HIP MoE layer (mirrors the reference's engines/ package paths)."""
