"""Import name of the package directory nano-vllm-speculative-decoding_amd/ (a directory name Python cannot import).

`import nvs_amd` loads that directory as the package `nvs_amd`; `import nvs_amd.layers.attention` and the other
submodules then resolve inside it.
"""
import importlib.util
import pathlib
import sys

_PKG_DIR = pathlib.Path(__file__).resolve().with_name("nano-vllm-speculative-decoding_amd")
_spec = importlib.util.spec_from_file_location(__name__, _PKG_DIR / "__init__.py",
                                               submodule_search_locations=[str(_PKG_DIR)])
_module = importlib.util.module_from_spec(_spec)
sys.modules[__name__] = _module
_spec.loader.exec_module(_module)
