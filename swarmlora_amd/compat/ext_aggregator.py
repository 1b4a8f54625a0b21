"""`import ext_aggregator` resolves here when swarmlora_amd.compat_path() is on sys.path:
the reference's extension module name bound to swarmlora_amd.ext_aggregator."""
from swarmlora_amd.ext_aggregator import *  # noqa: F401,F403
from swarmlora_amd import ext_aggregator as _impl

globals().update({k: getattr(_impl, k) for k in dir(_impl) if not k.startswith("__")})
