"""Engine-side helpers of the hot path (token sampling and speculative verification)."""
