"""Where julia1-rs_amd/build.py puts the built artefacts (kept in-tree so they travel with the repository)."""
import os

_LIB_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib")
SHARED = os.path.join(_LIB_DIR, "libjulia1_hip.so")
ARCHIVE = os.path.join(_LIB_DIR, "libjulia1_hip.a")
CALLER = os.path.join(_LIB_DIR, "jh_caller")
