"""Creator/follower sharing of one host copy of a streamed model between processes.

:class:`SharedOffloadSession` keeps the reference's public interface
(shared_offload.py:110-521). Every worker process constructs a session with
the same namespace and calls :meth:`~SharedOffloadSession.offload_from_profile`:

* the first process to create the namespace's control segment becomes the
  **creator**: it builds the model with its checkpoint factory, offloads it
  with the saved profile so every streamed label's block is packed into a named
  shared-memory segment, publishes the resident tensors as a
  :class:`~flextensor_amd.shm.SharedTensorStore` and its live profile, and
  marks the namespace ready;
* every other process is a **follower**: it waits for readiness, builds the
  model skeleton (normally on the ``meta`` device), copies the resident
  tensors out of the store onto its GPU, maps the creator's block segments
  (no host copy) and streams from them.

Shared blocks are pageable mappings. ``pinned_memory_mode="host_register"``
page-locks them in place (the reference's ``cudaHostRegister`` of SHM blocks,
shm/flexible_shm.py:832-848); otherwise their copies go through the staged
copy engine (pinned staging buffers filled by a host thread pool).

:class:`ShmCoordinator` is the election and readiness protocol (the role of
shm/coordinator.py:75-360): a control segment ``<ns>_c`` created atomically
(the creator is whoever publishes it first), holding the creator's state
(initializing, ready, failed), its process id, a heartbeat the creator
refreshes from a background thread, and the failure message. The live
profile is ``<ns>_p`` in the reference's length-prefixed bytes form
(state_handler.py:1457-1500).
"""

from __future__ import annotations

import hashlib
import logging
import math
import os
import re
import struct
import sys
import threading
import time
from collections.abc import Callable, Iterable
from dataclasses import dataclass, field
from typing import Any

import torch
from torch import nn

from .config import OffloadConfig
from .layout import DEFAULT_ALIGNMENT, plan_block
from .manager import DEFAULT_MANAGER_NAME, OffloadManager, get_offload_manager, release
from .profile import TensorManagerState, load_state, load_state_from_bytes, save_state_to_bytes
from .shm import SHM_DIR, SharedSegment, SharedTensorStore

LOGGER = logging.getLogger(__name__)

_NAMESPACE_RE = re.compile(r"[A-Za-z0-9][A-Za-z0-9_.-]{0,95}\Z")
_MANAGER_RE = re.compile(r"[A-Za-z0-9][A-Za-z0-9_.-]{0,63}\Z")

PROTOCOL_VERSION = 1
DEFAULT_KEEP_ALIVE_SECONDS = 30.0
_MAGIC = b"FTSC"
# magic, protocol version, state, failure message length, creator pid, heartbeat, created (wall-clock seconds)
_HEADER = struct.Struct("<4sIIIqdd")
_MESSAGE_OFFSET = 64
_CONTROL_BYTES = 4096
INITIALIZING, READY, FAILED = 1, 2, 3


class ShmCoordinatorError(RuntimeError):
    """Base class for failures of the shared initialization protocol."""


class ShmCreatorFailedError(ShmCoordinatorError):
    """Raised in followers when the creator published a failure."""

    def __init__(self, namespace: str, failure_message: str) -> None:
        self.namespace = namespace
        self.failure_message = failure_message
        super().__init__(f"Shared initialization for namespace '{namespace}' failed: "
                         f"{failure_message or 'creator initialization failed without details'}")


class ShmCreatorDiedError(ShmCoordinatorError):
    """Raised in followers when the creator's heartbeat expired (while initializing, or after it was ready)."""

    def __init__(self, namespace: str, creator_identity: int | None, *, after_ready: bool = False) -> None:
        self.namespace = namespace
        self.creator_identity = creator_identity
        self.after_ready = after_ready
        detail = "unknown" if creator_identity is None else str(creator_identity)
        if after_ready:
            super().__init__(f"Creator participant {detail} of shared namespace '{namespace}' has exited; its "
                             "segments are left from a finished run. Remove them with "
                             "SharedOffloadSession.cleanup_namespace before reusing the namespace")
        else:
            super().__init__(f"Creator participant {detail} died while initializing shared namespace '{namespace}'")


def control_segment_name(namespace: str) -> str:
    return f"{namespace}_c"


def profile_segment_name(namespace: str) -> str:
    return f"{namespace}_p"


class ShmCoordinator:
    """Election, readiness and failure publication for one namespace."""

    def __init__(self, namespace: str, keep_alive_seconds: float = DEFAULT_KEEP_ALIVE_SECONDS,
                 heartbeat_interval: float = 0.5) -> None:
        if keep_alive_seconds <= 0 or heartbeat_interval <= 0:
            raise ValueError("keep_alive_seconds and heartbeat_interval must be positive")
        self.namespace = namespace
        self.keep_alive_seconds = float(keep_alive_seconds)
        self.heartbeat_interval = float(heartbeat_interval)
        self._profile: SharedSegment | None = None
        self._stop = threading.Event()
        self._beat: threading.Thread | None = None
        self._write_lock = threading.Lock()  # the heartbeat thread and the owner both rewrite the header
        name = control_segment_name(namespace)
        now = time.time()
        try:
            self._control = SharedSegment(name, _CONTROL_BYTES, create=True, initializer=lambda buf: _HEADER.pack_into(
                buf, 0, _MAGIC, PROTOCOL_VERSION, INITIALIZING, 0, os.getpid(), now, now))
            self.is_creator = True
        except FileExistsError:
            self._control = SharedSegment(name)
            self.is_creator = False
            if self._control.size < _CONTROL_BYTES:
                self._control.close()
                raise ShmCoordinatorError(f"control segment of namespace '{namespace}' is truncated")
            magic, version = _HEADER.unpack_from(self._control.buf, 0)[:2]
            if magic != _MAGIC or version != PROTOCOL_VERSION:
                self._control.close()
                raise ShmCoordinatorError(f"namespace '{namespace}' uses another protocol "
                                          f"({magic!r} v{version}, this side v{PROTOCOL_VERSION})")
        if self.is_creator:
            self._beat = threading.Thread(target=self._heartbeat, name=f"ftx-heartbeat-{namespace}", daemon=True)
            self._beat.start()

    # -- header fields ------------------------------------------------------------------

    def _header(self) -> tuple[int, int, int, float]:
        _, _, state, msg_len, pid, beat, _ = _HEADER.unpack_from(self._control.buf, 0)
        return state, msg_len, pid, beat

    def _write(self, state: int | None = None, message: str | None = None, beat: float | None = None) -> None:
        with self._write_lock:
            buf = self._control.buf
            magic, version, cur_state, msg_len, pid, cur_beat, created = _HEADER.unpack_from(buf, 0)
            if message is not None:  # the message lands before the state that announces it
                raw = message.encode("utf-8", errors="replace")[: _CONTROL_BYTES - _MESSAGE_OFFSET]
                buf[_MESSAGE_OFFSET:_MESSAGE_OFFSET + len(raw)] = raw
                msg_len = len(raw)
            _HEADER.pack_into(buf, 0, magic, version, cur_state if state is None else state, msg_len, pid,
                              cur_beat if beat is None else beat, created)

    def _heartbeat(self) -> None:
        while not self._stop.wait(self.heartbeat_interval):
            try:
                self._write(beat=time.time())
            except (RuntimeError, ValueError):
                return  # the segment was closed

    # -- creator ------------------------------------------------------------------------

    def _require_creator(self) -> None:
        if not self.is_creator:
            raise RuntimeError("only the creator publishes to a shared namespace")

    def write_profile(self, state: TensorManagerState) -> None:
        """Publish the live profile (length-prefixed JSON) for followers."""
        self._require_creator()
        payload = save_state_to_bytes(state)

        def fill(buf: memoryview) -> None:
            buf[: len(payload)] = payload

        self._profile = SharedSegment(profile_segment_name(self.namespace), len(payload), create=True,
                                      initializer=fill)

    def notify_ready(self) -> None:
        self._require_creator()
        self._write(state=READY, beat=time.time())

    def mark_failed(self, error: BaseException) -> None:
        """Publish the creator's failure so waiting followers raise instead of timing out."""
        self._require_creator()
        self._write(state=FAILED, message=f"{type(error).__name__}: {error}", beat=time.time())

    # -- followers ----------------------------------------------------------------------

    def state(self) -> int:
        return self._header()[0]

    def is_creator_alive(self) -> bool:
        """Whether the creator's heartbeat is fresh (it beats from creation until the creator closes)."""
        return time.time() - self._header()[3] <= self.keep_alive_seconds

    def wait_for_ready(self, timeout: float | None = None, poll: float = 0.02) -> None:
        """Return once the creator is ready; raise when it failed, died or ``timeout`` passed.

        A ready namespace whose creator no longer beats is refused too: its
        segments are what a finished (or killed) run left behind, and a new
        run that joined them would read that run's weights
        (the reference refuses a generation with no live participant,
        shm/coordinator.py:75-360).
        """
        deadline = None if not timeout else time.monotonic() + timeout
        stale = 0
        while True:
            state, msg_len, pid, beat = self._header()
            if state == FAILED:
                msg = bytes(self._control.buf[_MESSAGE_OFFSET:_MESSAGE_OFFSET + msg_len]).decode("utf-8", "replace")
                raise ShmCreatorFailedError(self.namespace, msg)
            # a stale heartbeat must be seen on two polls in a row (a read racing a write is not proof)
            stale = stale + 1 if time.time() - beat > self.keep_alive_seconds else 0
            if state == READY and stale == 0:
                return
            if stale >= 2:
                raise ShmCreatorDiedError(self.namespace, pid, after_ready=state == READY)
            if deadline is not None and time.monotonic() > deadline:
                raise TimeoutError(f"timed out after {timeout} s waiting for the creator of namespace "
                                   f"'{self.namespace}'")
            time.sleep(poll)

    def read_profile(self) -> TensorManagerState:
        seg = SharedSegment(profile_segment_name(self.namespace))
        try:
            return load_state_from_bytes(bytes(seg.buf))
        finally:
            seg.close()

    def close(self) -> None:
        """Stop the heartbeat; the creator also removes the control and profile names."""
        self._stop.set()
        if self._beat is not None:
            self._beat.join()
            self._beat = None
        if self._profile is not None:
            self._profile.close()
            self._profile = None
        self._control.close()


def _normalize_options(namespace: object, wait_timeout: Any) -> tuple[str, float]:
    if not isinstance(namespace, str) or _NAMESPACE_RE.fullmatch(namespace) is None:
        raise ValueError("Shared offload namespace must be 1-96 POSIX-safe characters: letters, digits, '.', '_' or '-'")
    if isinstance(wait_timeout, bool):
        raise ValueError("Shared offload wait timeout must be a non-negative finite number")
    try:
        t = float(wait_timeout)
    except (TypeError, ValueError, OverflowError) as error:
        raise ValueError("Shared offload wait timeout must be a non-negative finite number") from error
    if not math.isfinite(t) or t < 0:
        raise ValueError("Shared offload wait timeout must be a non-negative finite number")
    return namespace, t


def _resident_parameter_names(model: nn.Module, names: Iterable[str]) -> list[str]:
    """The parameters among a state's GPU-resident names (shared_offload.py:87-107)."""
    params = dict(model.named_parameters(recurse=True, remove_duplicate=False))
    buffers = dict(model.named_buffers(recurse=True, remove_duplicate=False))
    wanted = list(names)
    unknown = sorted(set(wanted) - params.keys() - buffers.keys())
    if unknown:
        raise RuntimeError(f"Shared offload GPU tensor names are not registered by the final model: {unknown!r}")
    return [n for n in wanted if n in params]


def _set_parameter(model: nn.Module, name: str, param: nn.Parameter) -> None:
    owner, _, leaf = name.rpartition(".")
    setattr(model.get_submodule(owner) if owner else model, leaf, param)


def attach_streamed_blocks(model: nn.Module, state: TensorManagerState) -> list[SharedSegment]:
    """Rebind every streamed parameter to a view of its label's shared block (no copy).

    The follower's parameters supply shapes, dtypes and strides (they may be
    ``meta``); each label's tensors are laid out in the saved strategy order
    with the same 128-byte packing the creator used, and every alias of a
    parameter is rebound. Returns the mapped segments (close them after the
    model is released).
    """
    if not state.shm_block_name_map:
        raise ValueError("the profile names no shared blocks")
    params = dict(model.named_parameters(recurse=True, remove_duplicate=False))
    aliases: dict[int, list[str]] = {}
    for n, p in params.items():
        aliases.setdefault(id(p), []).append(n)
    segments: list[SharedSegment] = []
    try:
        for label, stats in state.load_strategy.items():
            if not stats:
                continue
            seen: set[int] = set()
            tensors: list[torch.Tensor] = []
            for t in stats:
                p = params.get(t.name)
                if p is None:
                    raise ValueError(f"streamed tensor {t.name!r} is not a parameter of the follower model")
                if id(p) not in seen:
                    seen.add(id(p))
                    tensors.append(p)
            slots, total = plan_block(tensors, DEFAULT_ALIGNMENT)
            seg = SharedSegment(state.shm_block_name_map[label])
            segments.append(seg)
            if seg.size < max(total, 1):
                raise ValueError(f"shared block of {label!r} holds {seg.size} bytes, its tensors need {total}")
            block = torch.frombuffer(seg.buf, dtype=torch.uint8, count=max(total, 1))
            for p, slot in zip(tensors, slots):
                new = nn.Parameter(slot.view(block), requires_grad=False)
                for n in aliases[id(p)]:
                    _set_parameter(model, n, new)
    except BaseException:
        segments.clear()  # rebound parameters may view them; mappings go with their last tensor
        raise
    return segments


@dataclass
class _LoadResources:
    """What one load holds until its cleanup succeeds."""

    manager_name: str | None = None
    store: SharedTensorStore | None = None
    coordinator: ShmCoordinator | None = None
    segments: list[SharedSegment] = field(default_factory=list)
    preserve_model: bool = False

    def close(self) -> None:
        if self.manager_name is not None:
            release(self.manager_name, preserve_model=self.preserve_model)
            self.manager_name = None
        if self.store is not None:
            self.store.close()
            self.store = None
        # follower mappings of the shared blocks: dropped, not closed (tensors may still view
        # them; each mapping goes away with its last tensor)
        self.segments.clear()
        if self.coordinator is not None:
            self.coordinator.close()
            self.coordinator = None


class SharedOffloadSession:
    """Shared offload managers of one worker process (shared_offload.py:110-521).

    Construct one session in every worker after spawning, with the same
    namespace; use it from the thread that constructed it.
    """

    def __init__(self, namespace: str, *, wait_timeout: Any = 300.0,
                 keep_alive_seconds: float = DEFAULT_KEEP_ALIVE_SECONDS) -> None:
        if sys.platform == "win32":
            raise NotImplementedError("Shared memory (SHM) is not supported on Windows")
        self.namespace, self.wait_timeout = _normalize_options(namespace, wait_timeout)
        self.keep_alive_seconds = float(keep_alive_seconds)
        self._resources: dict[str, _LoadResources] = {}
        self._loading: set[str] = set()
        self._pending_cleanup: dict[str, _LoadResources] = {}
        self._closed = False
        self._owner_pid = os.getpid()
        self._owner_thread = threading.get_ident()
        self.roles: dict[str, str] = {}

    @staticmethod
    def validate_options(namespace: object, *, wait_timeout: Any = 300.0) -> None:
        _normalize_options(namespace, wait_timeout)

    def _check_owner(self) -> None:
        if os.getpid() != self._owner_pid:
            raise RuntimeError("SharedOffloadSession cannot be used after fork; construct a new session inside "
                               "each worker process")
        if threading.get_ident() != self._owner_thread:
            raise RuntimeError(f"SharedOffloadSession belongs to thread {self._owner_thread}, but was accessed "
                               f"from thread {threading.get_ident()}")

    def namespace_for(self, name: str) -> str:
        """A compact namespace of its own for each named manager (shared_offload.py:173-180)."""
        if not isinstance(name, str) or _MANAGER_RE.fullmatch(name) is None:
            raise ValueError("Shared offload manager name must be 1-64 POSIX-safe characters: letters, digits, "
                             "'.', '_' or '-'")
        return "ft_" + hashlib.sha256(f"{self.namespace}\0{name}".encode()).hexdigest()[:12]

    @staticmethod
    def cleanup_namespace(namespace: str, *, manager_names: Iterable[str], timeout: Any = 60.0,
                          keep_alive_seconds: float = DEFAULT_KEEP_ALIVE_SECONDS) -> None:
        """Remove an abandoned run's segments (stop all workers first).

        A namespace whose creator heartbeat is fresh is live and is not
        touched (``ShmCoordinatorError`` once ``timeout`` has passed); a
        missing namespace is a no-op.
        """
        namespace, timeout = _normalize_options(namespace, timeout)
        if isinstance(manager_names, str):
            raise ValueError("manager_names must be an iterable of manager names, not a string")
        session = SharedOffloadSession(namespace)
        names = [session.namespace_for(n) for n in manager_names]
        if not names:
            raise ValueError("manager_names must not be empty")
        deadline = time.monotonic() + timeout
        for ns in dict.fromkeys(names):
            while True:
                try:
                    ctrl = SharedSegment(control_segment_name(ns))
                except FileNotFoundError:
                    live = False
                else:
                    try:
                        _, _, state, _, _, beat, _ = _HEADER.unpack_from(ctrl.buf, 0)
                        live = state != FAILED and time.time() - beat <= keep_alive_seconds
                    finally:
                        ctrl.close()
                if not live:
                    break
                if time.monotonic() >= deadline:
                    raise ShmCoordinatorError(f"namespace '{ns}' has a live creator; stop it before cleanup")
                time.sleep(0.25)
            prefix = f"{ns}_"
            for entry in os.listdir(SHM_DIR):
                if entry.startswith(prefix):
                    try:
                        os.unlink(os.path.join(SHM_DIR, entry))
                    except FileNotFoundError:
                        pass

    def offload_from_profile(
        self,
        profile_directory: str | os.PathLike[str],
        *,
        config: OffloadConfig,
        name: str = DEFAULT_MANAGER_NAME,
        creator_model_factory: Callable[[], nn.Module],
        follower_model_factory: Callable[[], nn.Module],
        materialize_device: torch.device | str | None = None,
        compile_fn: Callable[[nn.Module], Any] | None = None,
    ) -> nn.Module:
        """Elect a role and restore a model straight into its saved placement (shared_offload.py:200-340)."""
        self._check_owner()
        ns = self.namespace_for(name)
        if not config.enabled:
            raise ValueError("Shared offload requires OffloadConfig.enabled=True")
        if config.transfer_mode != "allocation_block_transfer":
            raise ValueError("Shared offload requires OffloadConfig.transfer_mode='allocation_block_transfer'")
        if self._closed:
            raise RuntimeError("Shared offload session is closed")
        if name in self._resources or name in self._loading or name in self._pending_cleanup:
            raise RuntimeError(f"Shared offload manager {name!r} has already been loaded")
        self._loading.add(name)
        res = _LoadResources()
        ready = False
        try:
            cfg = config.model_copy(update={"shm_enabled": True, "shm_namespace": ns,
                                            "shm_wait_timeout": self.wait_timeout})
            manager = get_offload_manager(name)
            if manager.model is not None:
                raise RuntimeError(f"offload manager {name!r} already manages a model")
            res.coordinator = ShmCoordinator(ns, keep_alive_seconds=self.keep_alive_seconds)
            role = "creator" if res.coordinator.is_creator else "follower"
            LOGGER.info("shared offload: role=%s manager=%s namespace=%s", role, name, ns)
            if res.coordinator.is_creator:
                model = self._load_creator(res, manager, cfg, name, profile_directory, creator_model_factory,
                                           compile_fn)
            else:
                model = self._load_follower(res, manager, cfg, name, follower_model_factory, materialize_device,
                                            compile_fn)
            self._resources[name] = res
            self.roles[name] = role
            if res.coordinator.is_creator:
                res.coordinator.notify_ready()
                ready = True
            return model
        except BaseException as error:
            if res.coordinator is not None and res.coordinator.is_creator and not ready:
                try:
                    res.coordinator.mark_failed(error)
                except BaseException:
                    LOGGER.exception("could not publish the creator's failure for namespace %s", ns)
            try:
                res.close()
            except BaseException:
                self._pending_cleanup[name] = res
                LOGGER.exception("cleanup of shared offload manager %s failed; retry with close()", name)
            raise
        finally:
            self._loading.discard(name)

    def _load_creator(self, res: _LoadResources, manager: OffloadManager, cfg: OffloadConfig, name: str,
                      profile_directory: str | os.PathLike[str], factory: Callable[[], nn.Module],
                      compile_fn: Callable[[nn.Module], Any] | None) -> nn.Module:
        disk_state = load_state(os.fspath(profile_directory))
        model = factory()
        res.manager_name = name
        manager.offload(model, cfg, state=disk_state, compile_fn=compile_fn)
        live = manager.state()
        res.store = SharedTensorStore.create_from_model(
            cfg.shm_namespace, model, parameter_names=_resident_parameter_names(model, live.gpu_tensors_names))
        assert res.coordinator is not None
        res.coordinator.write_profile(live)
        return model

    def _load_follower(self, res: _LoadResources, manager: OffloadManager, cfg: OffloadConfig, name: str,
                       factory: Callable[[], nn.Module], device: torch.device | str | None,
                       compile_fn: Callable[[nn.Module], Any] | None) -> nn.Module:
        assert res.coordinator is not None
        res.coordinator.wait_for_ready(timeout=self.wait_timeout or None)
        live = res.coordinator.read_profile()
        model = factory()
        _resident_parameter_names(model, live.gpu_tensors_names)
        res.store = SharedTensorStore.attach(cfg.shm_namespace)
        target = device if device is not None else torch.device("cuda", cfg.gpu_device)
        res.store.materialize_into(model, device=target)
        res.segments = attach_streamed_blocks(model, live)
        res.manager_name = name
        manager.offload(model, cfg, state=live, compile_fn=compile_fn, load_from_shm=True)
        return model

    def close(self, *, preserve_models: bool = False) -> None:
        """Release the loaded managers in reverse order; idempotent, retryable after a failure."""
        self._check_owner()
        if self._closed and not self._resources and not self._pending_cleanup:
            return
        self._closed = True
        for name in reversed(list(self._resources)):
            res = self._resources.pop(name)
            res.preserve_model = preserve_models
            self._pending_cleanup[name] = res
        first: BaseException | None = None
        for name in list(self._pending_cleanup):
            try:
                self._pending_cleanup[name].close()
            except BaseException as error:
                first = first or error
            else:
                del self._pending_cleanup[name]
        if first is not None:
            raise first

    def __enter__(self) -> "SharedOffloadSession":
        return self

    def __exit__(self, exc_type: object, exc: object, tb: object) -> None:
        try:
            self.close()
        except BaseException:
            if exc_type is None:
                raise
            LOGGER.exception("closing the shared offload session failed while another exception was in flight")


__all__ = ["SharedOffloadSession", "ShmCoordinator", "ShmCoordinatorError", "ShmCreatorDiedError",
           "ShmCreatorFailedError", "attach_streamed_blocks"]
