"""Deployment loading for the ``fa`` op group.

Contract kept from the reference facade (``CustomOps.build`` /
``load_precompiled`` / ``load``, __init__.py:654-1011, and ``FAOps``,
recsys.py:165-202): an offline build that publishes the library together with
a metadata sidecar; a precompiled load that validates everything it can
BEFORE the library is opened and then verifies the registered operator
(schema, Meta kernel); a strict mode in which nothing is compiled; and one
owner per dispatcher operator per process (a second library for the same
operator, a modified file, or an operator registered behind the loader's
back fails closed).

This module's own design for that contract:

* The sidecar is a *sealed artifact manifest* (``ARTIFACT_FORMAT``) with four
  sections — ``contract`` (operator namespace, schemas, Meta ops, C ABI),
  ``runtime`` (torch major.minor, HIP major), ``targets`` (gfx names) and
  ``provenance`` (sources digest, flags, compiler) — plus ``payload`` (file
  name, size, SHA-256). ``seal`` is the SHA-256 of the canonical JSON of all
  of them, so any edit of the sidecar is caught before its content is
  trusted.
* Validation is a table of named checks (``_CHECKS``), each comparing one
  section with what this process expects and returning a message, so the
  error says which section disagreed and how.
* Ownership is an explicit state machine per operator in ``_REGISTRY``:
  a claim is ``reserved`` before the library is opened, ``live`` once its
  operator verified, ``broken`` if anything failed in between (the process
  must be restarted to retry, as a half-registered operator cannot be
  removed from the dispatcher).
"""
from __future__ import annotations

import dataclasses
import fcntl
import hashlib
import json
import os
import re
import subprocess
import tempfile
import threading
from pathlib import Path
from typing import Callable, Optional

import torch

from . import _lib, build as _build, fa

ARTIFACT_FORMAT = "custom_ops_amd.artifact/2"
GROUP_VERSION = "1"


class CustomOpsError(RuntimeError):
    """Load/build failure (the reference's exception type name, __init__.py:71)."""


# ── artifact manifest ─────────────────────────────────────────────────────────

def _canonical(obj) -> bytes:
    return json.dumps(obj, sort_keys=True, separators=(",", ":")).encode()


def seal_of(manifest: dict) -> str:
    """SHA-256 over every section except the seal itself."""
    return hashlib.sha256(_canonical({k: v for k, v in manifest.items() if k != "seal"})).hexdigest()


def _digest_file(path: Path) -> str:
    h = hashlib.sha256()
    with path.open("rb") as f:
        while True:
            block = f.read(1 << 20)
            if not block:
                return h.hexdigest()
            h.update(block)


def _runtime_section() -> dict:
    """What a library built by this process's toolchain needs from a loading process."""
    hip = (getattr(torch.version, "hip", None) or "").split(".")[0]
    return {"torch": ".".join(torch.__version__.split("+")[0].split(".")[:2]), "hip": hip}


_GFX = re.compile(r"gfx[0-9a-f]{3,4}")


def _targets(value) -> list:
    """Sorted unique gfx names from 'gfx950;gfx942' or a list; rejects malformed names."""
    names = value.split(";") if isinstance(value, str) else list(value)
    out = sorted({str(n).strip() for n in names if str(n).strip()})
    bad = [n for n in out if not _GFX.fullmatch(n)]
    if bad:
        raise CustomOpsError(f"invalid offload target(s) {bad} (expected names like 'gfx950')")
    return out


def _visible_archs() -> set:
    """gfx names of the GPUs this process can see (empty without a GPU)."""
    if not torch.cuda.is_available():
        return set()
    return {torch.cuda.get_device_properties(i).gcnArchName.split(":")[0]
            for i in range(torch.cuda.device_count())}


def _registered_schema(qualified: str) -> Optional[str]:
    try:
        found = torch._C._jit_get_schemas_for_operator(qualified)
    except RuntimeError:
        return None
    return str(found[0]) if found else None


@dataclasses.dataclass(frozen=True)
class _Expectation:
    """What the loading process requires of an artifact."""
    contract: dict
    runtime: dict
    visible: frozenset


def _section_diff(name: str, got, want) -> Optional[str]:
    if got == want:
        return None
    if isinstance(got, dict) and isinstance(want, dict):
        keys = sorted(set(got) | set(want))
        diff = [f"{k}: artifact={got.get(k)!r} process={want.get(k)!r}"
                for k in keys if got.get(k) != want.get(k)]
        return f"{name} mismatch ({'; '.join(diff)})"
    return f"{name} mismatch: artifact={got!r} process={want!r}"


def _check_format(md: dict, exp: _Expectation, lib: Path) -> Optional[str]:
    if md.get("format") != ARTIFACT_FORMAT:
        return f"format mismatch: artifact={md.get('format')!r} process={ARTIFACT_FORMAT!r}"
    missing = [k for k in ("contract", "runtime", "targets", "provenance", "payload", "seal")
               if k not in md]
    return f"sidecar lacks section(s) {missing}" if missing else None


def _check_seal(md: dict, exp: _Expectation, lib: Path) -> Optional[str]:
    if not isinstance(md["seal"], str) or md["seal"] != seal_of(md):
        return "sidecar seal is broken (the metadata was edited after the build)"
    return None


def _check_contract(md: dict, exp: _Expectation, lib: Path) -> Optional[str]:
    return _section_diff("contract", md["contract"], exp.contract)


def _check_runtime(md: dict, exp: _Expectation, lib: Path) -> Optional[str]:
    return _section_diff("runtime", md["runtime"], exp.runtime)


def _check_targets(md: dict, exp: _Expectation, lib: Path) -> Optional[str]:
    t = md["targets"]
    if not isinstance(t, list) or not t or t != _targets(t):
        return "targets must be a non-empty sorted list of gfx names"
    uncovered = sorted(exp.visible - set(t))
    if uncovered:
        return f"target mismatch: the visible GPU(s) {uncovered} are not among the built {t}"
    return None


def _check_payload(md: dict, exp: _Expectation, lib: Path) -> Optional[str]:
    pl = md["payload"]
    if not isinstance(pl, dict) or pl.get("file") != lib.name:
        return f"payload names {pl.get('file') if isinstance(pl, dict) else pl!r}, not {lib.name!r}"
    size = lib.stat().st_size
    if type(pl.get("bytes")) is not int or pl["bytes"] != size:
        return f"payload size mismatch: sidecar {pl.get('bytes')!r} bytes, file {size}"
    if pl.get("sha256") != _digest_file(lib):
        return "payload digest mismatch: the library file differs from the one built"
    return None


_CHECKS: tuple = (
    ("format", _check_format),
    ("seal", _check_seal),
    ("contract", _check_contract),
    ("runtime", _check_runtime),
    ("targets", _check_targets),
    ("payload", _check_payload),
)


# ── operator ownership ────────────────────────────────────────────────────────

@dataclasses.dataclass
class _Claim:
    path: Path
    identity: tuple          # (st_dev, st_ino, sha256)
    state: str = "reserved"  # reserved -> live | broken
    reason: str = ""


_REGISTRY: dict = {}         # qualified op name -> _Claim
_LOCK = threading.RLock()


def _identity(path: Path) -> tuple:
    st = path.stat()
    return (st.st_dev, st.st_ino, _digest_file(path))


def _claim(ops: list, path: Path, identity: tuple) -> list:
    """Reserve ``ops`` for the library at ``path`` or raise; returns the claims
    (existing live ones are reused: loading the same file twice is idempotent)."""
    claims = []
    for op in ops:
        c = _REGISTRY.get(op)
        if c is None:
            if _registered_schema(op) is not None:
                raise CustomOpsError(
                    f"{op} is registered outside this loader (untracked library); "
                    "start a fresh process")
            continue
        if c.identity[:2] == identity[:2] and c.identity[2] != identity[2]:
            raise CustomOpsError(f"{c.path} changed on disk after it was loaded; "
                                 "start a fresh process")
        if c.identity != identity:
            raise CustomOpsError(f"{op} is already served by {c.path}; a second library "
                                 "(another build or a copy) cannot serve it in this process")
        if c.state == "broken":
            raise CustomOpsError(f"an earlier load of {c.path} failed midway ({c.reason}); "
                                 "start a fresh process")
        claims.append(c)
    if len(claims) == len(ops):
        return claims
    new = _Claim(path=path, identity=identity)
    for op in ops:
        _REGISTRY.setdefault(op, new)
    return [_REGISTRY[op] for op in ops]


def _loaded_identities() -> set:
    return {c.identity[:2] for c in _REGISTRY.values()}


# ── the op group ──────────────────────────────────────────────────────────────

class FAOps:
    """The ``fa`` op group (reference ``FAOps``, recsys.py:165-202)."""

    namespace = fa.NAMESPACE
    so_name = "libmi355_fa"
    ops = {fa.OP_NAME: fa.SCHEMA}
    meta_ops = (fa.OP_NAME,)
    default_targets = ("gfx950",)

    def __init__(self, *, allow_jit: bool = True) -> None:
        self._allow_jit = True
        self._library: Optional[Path] = None
        self._sidecar: Optional[Path] = None
        self._error: Optional[str] = None
        self.configure(allow_jit=allow_jit)

    # policy
    @property
    def allow_jit(self) -> bool:
        """Whether load() may compile the in-tree library (hipcc)."""
        return self._allow_jit

    @allow_jit.setter
    def allow_jit(self, value: bool) -> None:
        self.configure(allow_jit=value)

    def configure(self, *, allow_jit: bool) -> "FAOps":
        if not isinstance(allow_jit, bool):
            raise TypeError("allow_jit must be a bool")
        self._allow_jit = allow_jit
        return self

    def disable_jit(self) -> "FAOps":
        return self.configure(allow_jit=False)

    # state
    @property
    def library_path(self) -> Optional[Path]:
        return self._library

    @property
    def metadata_path(self) -> Optional[Path]:
        return self._sidecar

    def is_available(self) -> bool:
        return self._library is not None

    def load_error(self) -> Optional[str]:
        return self._error

    # contract
    def _qualified(self) -> list:
        return sorted(f"{self.namespace}::{op}" for op in self.ops)

    def contract(self) -> dict:
        return {"namespace": self.namespace,
                "schemas": {f"{self.namespace}::{op}": f"{self.namespace}::{schema}"
                            for op, schema in sorted(self.ops.items())},
                "meta_ops": sorted(self.meta_ops),
                "abi": _lib.ABI_VERSION,
                "group_version": GROUP_VERSION}

    def _expectation(self) -> _Expectation:
        return _Expectation(self.contract(), _runtime_section(), frozenset(_visible_archs()))

    # offline build
    def _provenance(self, targets: list, extra: list) -> dict:
        h = hashlib.sha256()
        csrc = Path(_build.SRC).parent
        for src in [Path(_build.SRC), *sorted(csrc.glob("*.h")), *sorted(csrc.glob("*.inc")),
                    *sorted(Path(_build.INCLUDE).glob("*.h"))]:
            h.update(src.name.encode() + b"\0" + src.read_bytes())
        flags = [f for f in _build.HIPCC_FLAGS if not f.startswith("--offload-arch=")] + extra
        try:
            ver = subprocess.run([_build.hipcc(), "--version"], capture_output=True, text=True,
                                 timeout=60).stdout.strip().splitlines()
        except (OSError, subprocess.SubprocessError):
            ver = []
        return {"sources_sha256": h.hexdigest(), "flags": flags,
                "compiler": next((l for l in ver if "version" in l.lower()), "")}

    def build(self, output_directory, *, offload_arch: Optional[str] = None,
              extra_flags=(), verbose: bool = False) -> Path:
        """Compile ``<so_name>.so`` for the targets and publish its sealed sidecar
        ``<so_name>.so.json`` next to it, without loading it. hipcc
        cross-compiles, so no GPU is needed. Deploy both files together."""
        targets = _targets(offload_arch or list(self.default_targets))
        if not targets:
            raise CustomOpsError("no offload target given")
        extra = []
        for f in extra_flags:
            if not isinstance(f, str) or not f.strip() or "\n" in f:
                raise CustomOpsError(f"invalid extra flag {f!r}")
            extra.append(f)
        out = Path(output_directory).expanduser().resolve()
        out.mkdir(parents=True, exist_ok=True)
        library = out / f"{self.so_name}.so"
        sidecar = Path(str(library) + ".json")
        with _LOCK, open(out / f".{self.so_name}.build.lock", "a") as lockf:
            fcntl.flock(lockf, fcntl.LOCK_EX)
            try:
                if library.exists() and (library.stat().st_dev, library.stat().st_ino) \
                        in _loaded_identities():
                    raise CustomOpsError(
                        f"cannot overwrite a library loaded in this process: {library}")
                before = self._provenance(targets, extra)
                with tempfile.TemporaryDirectory(prefix=".build-", dir=out) as tmp:
                    product = Path(tmp) / library.name
                    try:   # compiles and checks the device assembly (isa_check)
                        _build.compile_checked(
                            str(product), [*before["flags"], *[f"--offload-arch={t}" for t in targets]],
                            verbose=verbose)
                    except RuntimeError as e:
                        raise CustomOpsError(str(e)) from e
                    if self._provenance(targets, extra) != before:
                        raise CustomOpsError("sources changed during the build; nothing published")
                    manifest = {"format": ARTIFACT_FORMAT, "contract": self.contract(),
                                "runtime": _runtime_section(), "targets": targets,
                                "provenance": before,
                                "payload": {"file": library.name,
                                            "bytes": product.stat().st_size,
                                            "sha256": _digest_file(product)}}
                    manifest["seal"] = seal_of(manifest)
                    staged = Path(tmp) / "sidecar.json"
                    staged.write_text(json.dumps(manifest, sort_keys=True, indent=2) + "\n")
                    os.replace(product, library)
                    os.replace(staged, sidecar)
            finally:
                fcntl.flock(lockf, fcntl.LOCK_UN)
        return library

    # loading
    def _validate(self, library: Path, sidecar: Path) -> None:
        try:
            md = json.loads(sidecar.read_text())
        except (OSError, ValueError) as e:
            raise CustomOpsError(f"cannot read sidecar {sidecar}: {e}") from e
        if not isinstance(md, dict):
            raise CustomOpsError(f"sidecar {sidecar} is not a JSON object")
        exp = self._expectation()
        for name, check in _CHECKS:
            msg = check(md, exp, library)
            if msg:
                raise CustomOpsError(f"{name} check: {msg}")

    def _verify_registered(self) -> None:
        for qualified, schema in self.contract()["schemas"].items():
            got = _registered_schema(qualified)
            if got != schema:
                raise CustomOpsError(f"registered schema {got!r} differs from the contract {schema!r}")
        for op in self.meta_ops:
            if not torch._C._dispatch_has_kernel_for_dispatch_key(f"{self.namespace}::{op}", "Meta"):
                raise CustomOpsError(f"no Meta (fake) kernel for {self.namespace}::{op}")

    def _bind(self, library: Path, prevalidated: Callable[[], None]) -> None:
        """Claim the operators, open the library, register and verify, in that order."""
        prevalidated()
        identity = _identity(library)
        claims = _claim(self._qualified(), library, identity)
        if all(c.state == "live" for c in claims):
            return
        try:
            _lib.load(str(library))
            fa.register()
            self._verify_registered()
        except Exception as e:
            for c in claims:
                c.state, c.reason = "broken", str(e)
            raise
        for c in claims:
            c.state = "live"

    def load_precompiled(self, library_path, metadata_path=None) -> "FAOps":
        """Validate a deployed library and its sidecar (default ``<library>.json``),
        then load it. Switches this group to strict mode (no compiling)."""
        with _LOCK:
            self._allow_jit = False
            self._library = None
            try:
                library = Path(library_path).expanduser().resolve(strict=True)
                if not library.is_file():
                    raise CustomOpsError(f"not a file: {library}")
                sidecar = Path(metadata_path if metadata_path is not None
                               else str(Path(library_path).expanduser()) + ".json")
                sidecar = sidecar.expanduser().resolve(strict=True)
                self._validate(library, sidecar)
                stamp = library.stat()

                def unchanged():
                    now = library.stat()
                    if (now.st_ino, now.st_size, now.st_mtime_ns) != \
                            (stamp.st_ino, stamp.st_size, stamp.st_mtime_ns):
                        raise CustomOpsError(f"{library} changed while it was being validated")
                self._bind(library, unchanged)
                self._library, self._sidecar, self._error = library, sidecar, None
            except Exception as e:
                self._error = str(e)
                raise CustomOpsError(f"[FAOps] precompiled load failed (JIT disabled): {e}") from e
        return self

    def load(self) -> "FAOps":
        """Development path: the in-tree library, compiled with hipcc when it is
        missing and ``allow_jit`` is True."""
        with _LOCK:
            if self._library is not None:
                return self
            if not self._allow_jit:
                self._error = ("JIT is disabled for FAOps; call load_precompiled("
                               "library_path, metadata_path=None) before load()")
                raise CustomOpsError(self._error)
            try:
                path = Path(_build.lib_path())
                if not path.exists():
                    _build.build()
                path = path.resolve(strict=True)
                self._bind(path, lambda: None)
                self._library, self._sidecar, self._error = path, None, None
            except Exception as e:
                self._error = str(e)
                raise CustomOpsError(f"[FAOps] load failed: {e}") from e
        return self
