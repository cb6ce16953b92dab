"""Phase flag read by HybridMoE.forward (nano_ktrans/utils/context.py:5-32)."""
from dataclasses import dataclass


@dataclass
class Context:
    is_prefill: bool = False


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_prefill: bool, *args, **kwargs) -> None:
    global _CONTEXT
    _CONTEXT = Context(bool(is_prefill))


def reset_context() -> None:
    global _CONTEXT
    _CONTEXT = Context()
