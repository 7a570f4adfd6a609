"""Model integrations (reskv/models/__init__.py): ``ResKVForCausalLM`` loads on first use,
so importing the package needs neither transformers nor the HIP library."""

__all__ = ["ResKVForCausalLM"]


def __getattr__(name):
    if name == "ResKVForCausalLM":
        from .llama import ResKVForCausalLM

        return ResKVForCausalLM
    raise AttributeError(name)
