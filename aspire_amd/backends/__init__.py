"""Backend-side pieces of the hot path: page selectors and dump-variant specs."""
