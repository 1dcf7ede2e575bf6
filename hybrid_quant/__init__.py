"""Nemotron-H-8B decode quantization helpers under the reference's import paths.

`hybrid_quant.<name>` is the module `layer_quant_amd.<name>` itself (one module object, so
attributes set by the patch functions are shared), for the names the reference's drivers import:
int4_8b_attention, mamba_state_8b_kernel, nemotron_8b_decode_eval, data, env.
"""
import importlib
import sys

_ALIASED = ("env", "int4_8b_attention", "mamba_state_8b_kernel", "nemotron_8b_decode_eval", "data")


def __getattr__(name):
    if name in _ALIASED:
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)


_ORIGINAL_SPECS = {}


class _AliasFinder:
    """Resolves `hybrid_quant.<name>` to the already-importable `layer_quant_amd.<name>`."""

    @classmethod
    def find_spec(cls, fullname, path=None, target=None):
        prefix = __name__ + "."
        if not fullname.startswith(prefix) or fullname[len(prefix):] not in _ALIASED:
            return None
        import importlib.util

        return importlib.util.spec_from_loader(fullname, cls)

    @staticmethod
    def create_module(spec):
        module = importlib.import_module("layer_quant_amd." + spec.name.rsplit(".", 1)[1])
        sys.modules[spec.name] = module
        _ORIGINAL_SPECS[spec.name] = module.__spec__
        return module

    @staticmethod
    def exec_module(module):
        # the import machinery stamped the alias spec on the shared module; keep the real one
        for alias, original in list(_ORIGINAL_SPECS.items()):
            if sys.modules.get(alias) is module:
                module.__spec__ = original


if not any(f is _AliasFinder for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasFinder)
