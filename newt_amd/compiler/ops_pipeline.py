"""Cross-iteration software pipeline for nl.dot inside loops (placeholder)."""


class DotPipeline:
    pass
