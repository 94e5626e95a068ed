"""Loading the PluggableDevice adapter into TensorFlow, mirroring the
reference's loader (python/_loader.py:79-130: find the plugin library next
to the package, then load_pluggable_device_library; python/__init__.py:
66-75 loads it on import and warns on failure).

libtfma_tf.so exports SE_InitPlugin (device "AMDGPU"), TF_InitKernel (the
hot-path kernels and the op definitions of MusaBiasAddRelu, MusaAddV2Relu,
MusaShiftedAffineMap, MusaResourceApplyAdamMixed and
MusaGroupedResourceApplyAdam) and TF_InitGraph (the fusion and Adam-grouping
rewrite as a Grappler plugin optimizer).  TensorFlow is imported only when
load_plugin() is called.
"""
import os

PLUGIN_LIBRARY = "libtfma_tf.so"
DEVICE_TYPE = "AMDGPU"

_loaded_path = None


def find_plugin_library():
    """Path of libtfma_tf.so: $TFMA_PLUGIN_PATH if set, else next to this
    package.  Raises FileNotFoundError listing the places searched."""
    here = os.path.dirname(os.path.abspath(__file__))
    candidates = []
    env = os.environ.get("TFMA_PLUGIN_PATH")
    if env:
        candidates.append(env if env.endswith(".so") else os.path.join(env, PLUGIN_LIBRARY))
    candidates.append(os.path.join(here, PLUGIN_LIBRARY))
    for path in candidates:
        if os.path.exists(path):
            return os.path.normpath(path)
    searched = "\n".join(f"  - {os.path.normpath(p)}" for p in candidates)
    raise FileNotFoundError(f"plugin library '{PLUGIN_LIBRARY}' not found; searched:\n"
                            f"{searched}\nBuild it with `make -C "
                            "tensorflow_musa_extension_amd/csrc`.")


def load_plugin():
    """Loads the plugin into TensorFlow once (device, kernels, op
    definitions, graph optimizer) and returns its path."""
    global _loaded_path
    if _loaded_path is not None:
        return _loaded_path
    path = find_plugin_library()
    try:
        from tensorflow.python.framework.load_library import load_pluggable_device_library
    except ImportError as e:
        raise RuntimeError("TensorFlow with the PluggableDevice loader "
                           "(load_pluggable_device_library) is required to load "
                           f"{PLUGIN_LIBRARY}") from e
    load_pluggable_device_library(path)
    _loaded_path = path
    return path


def is_plugin_loaded():
    return _loaded_path is not None


def get_devices():
    """TensorFlow's physical devices of the plugin's type."""
    import tensorflow as tf
    return tf.config.list_physical_devices(DEVICE_TYPE)
