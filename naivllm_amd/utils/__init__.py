from naivllm_amd.utils.context import Context, get_context, reset_context, set_context

__all__ = ["Context", "get_context", "reset_context", "set_context"]
