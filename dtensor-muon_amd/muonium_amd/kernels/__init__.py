from .gram import gram, gram_

__all__ = ["gram", "gram_"]
