"""ResKV compressed-KV hot path for AMD Instinct MI355X (gfx950).

Same public surface as the reference package ``reskv`` for this path
(``reskv/__init__.py``): ``ResKVKernelConfig``, ``compress``, ``attention`` and
``ResKVForCausalLM``, plus the submodules ``config``, ``tensors``,
``compression``, ``cache``, ``models``, ``_attention`` and ``_extension``.
Importing the package imports neither torch nor the HIP library; both load on
first use of an operator.
"""

from .config import KernelPlan, ResKVKernelConfig

__version__ = "0.1.0"
__all__ = ["ResKVKernelConfig", "KernelPlan", "ResKVForCausalLM", "compress", "attention"]


def __getattr__(name):
    if name == "compress":
        from .compression import compress

        return compress
    if name == "attention":
        from ._attention import attention

        return attention
    if name == "ResKVForCausalLM":
        from .models.llama import ResKVForCausalLM

        return ResKVForCausalLM
    raise AttributeError(name)
