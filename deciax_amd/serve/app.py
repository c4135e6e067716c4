"""HTTP service for `/v1/systemone` over the HIP decision path.

The routes, bodies, limits and status codes are those of the reference's server
(src/deciax/serve/app.py:100-423): `POST /v1/systemone`, `POST /v1/systemone/batch` and
`GET /health`; 400 for malformed bodies, 401 without the bearer token, 404 / 405 for unknown
routes, 411 / 413 for missing or oversized bodies, 422 for requests the model rejects (its
ValueError), 500 for a failed inference and 503 when every admission slot is taken. `Service`
holds that logic apart from the HTTP framework; a stdlib `ThreadingHTTPServer` adapts it. The
device forward itself is serialised by each engine's lock, as the reference's is.
"""

from __future__ import annotations

import hmac
import json
import logging
import threading
import time
from collections.abc import Callable, Mapping
from dataclasses import dataclass, field
from http.server import BaseHTTPRequestHandler, ThreadingHTTPServer
from pathlib import Path
from typing import Any

from deciax_amd.serve.protocol import (
    DEFAULT_LIMITS,
    MAX_BODY_BYTES,
    SURROGATE_DETAIL,
    RequestError,
    check_batch,
    check_request,
    has_lone_surrogate,
    strict_view,
    with_confidence,
)

log = logging.getLogger("deciax_amd.serve")

# Body fields the reference refuses rather than ignores (src/deciax/serve/app.py:67-75)
HOOK_FIELDS = ("hooks", "on_predict_start", "on_predict_end", "hooks_raise", "hooks_timeout")
UNSUPPORTED = ("task", "lang", "lang_guess", "min_confidence", "images", "videos", "media_kwargs")
UNSUPPORTED_BATCH = ("batch_size", "sort_by_length", "diagnostics")


@dataclass
class Response:
    status: int
    payload: Any
    headers: dict[str, str] = field(default_factory=dict)


def _error(status: int, detail: str, headers: dict[str, str] | None = None) -> Response:
    return Response(status, {"detail": detail}, headers or {})


class Service:
    """Protocol logic over loaded deciders (objects with `decide` / `decide_batch`)."""

    def __init__(self, deciders: Mapping[str, Any], default_model: str, *, api_key: str | None = None,
                 max_concurrent: int = 16, jev_strict: bool = False, device: str = "unknown") -> None:
        if default_model not in deciders:
            raise ValueError(f"default model {default_model!r} is not loaded")
        if max_concurrent < 1:
            raise ValueError("max_concurrent must be at least 1")
        self.deciders = dict(deciders)
        self.default_model = default_model
        self.jev_strict = jev_strict
        self.device = device
        self._token = ("Bearer " + api_key).encode() if api_key else None
        self._slots = threading.BoundedSemaphore(max_concurrent)

    def handle(self, method: str, path: str, headers: Mapping[str, str], body: bytes) -> Response:
        route = path.split("?", 1)[0].rstrip("/") or "/"
        auth = headers.get("authorization")
        if route == "/health":
            return Response(200, self._health(auth)) if method == "GET" else _error(405, "Method Not Allowed")
        endpoints: dict[str, Callable[[bytes], Response]] = {"/v1/systemone": self._one,
                                                             "/v1/systemone/batch": self._batch}
        endpoint = endpoints.get(route)
        if endpoint is None:
            return _error(404, "Not Found")
        if method != "POST":
            return _error(405, "Method Not Allowed")
        if not self.authorized(auth):
            return _error(401, "invalid or missing bearer token")
        if not self._slots.acquire(blocking=False):
            return _error(503, "server busy, try again later", {"Retry-After": "1"})
        try:
            return endpoint(body)
        except RequestError as e:
            return _error(e.status, e.detail)
        finally:
            self._slots.release()

    def authorized(self, authorization: str | None) -> bool:
        if self._token is None:
            return True
        return hmac.compare_digest((authorization or "").encode("utf-8", "surrogateescape"), self._token)

    def _health(self, authorization: str | None) -> dict[str, Any]:
        if not self.authorized(authorization):
            return {"status": "ok"}
        return {"status": "ok", "loaded": sorted(self.deciders), "default_model": self.default_model,
                "device": self.device}

    def _one(self, raw: bytes) -> Response:
        body = _parse(raw)
        if not isinstance(body, dict) or "questions" not in body:
            raise RequestError(400, "request body must be an object with a 'questions' field")
        decider = self.deciders[self.model_for(body.get("model"))]
        state, questions = body.get("state"), body["questions"]
        check_request(state, questions, DEFAULT_LIMITS)
        _refuse(body, UNSUPPORTED)
        if has_lone_surrogate(body):
            raise RequestError(400, SURROGATE_DETAIL)
        budgets = _budgets(body, _token_cap(decider))
        result, ms = self._run(lambda: decider.decide(state, questions, **budgets))
        return Response(200, self._finish(result), _timing(ms))

    def _batch(self, raw: bytes) -> Response:
        body = _parse(raw)
        if not isinstance(body, dict) or "questions" not in body or "states" not in body:
            raise RequestError(400, "request body must be an object with 'states' and 'questions' fields")
        decider = self.deciders[self.model_for(body.get("model"))]
        states, questions = body["states"], body["questions"]
        check_batch(states, questions, DEFAULT_LIMITS)
        _refuse(body, UNSUPPORTED + UNSUPPORTED_BATCH)
        if has_lone_surrogate(body):
            raise RequestError(400, SURROGATE_DETAIL)
        budgets = _budgets(body, _token_cap(decider))
        results, ms = self._run(lambda: decider.decide_batch(states, questions, **budgets))
        usage = {key: sum(r["usage"].get(key, 0) for r in results) for key in ("input_tokens", "output_tokens")}
        return Response(200, {"results": [self._finish(r) for r in results], "total_usage": usage}, _timing(ms))

    def model_for(self, requested: Any) -> str:
        """The loaded model a request's `model` field selects. Absent or unknown names let the server
        choose (the default model); a loaded name selects it; a registered shape this server has not
        loaded, or anything that looks like a path, is a 422."""
        if not requested:
            return self.default_model
        text = str(requested).strip()
        if text in self.deciders:
            return text
        from deciax_amd import gemma

        if text in gemma.CONFIGS:
            raise RequestError(422, f"model {text!r} is not loaded; this server serves {sorted(self.deciders)}")
        if text[:1] in ".~" or "/" in text or "\\" in text:
            raise RequestError(422, f"unknown model {text!r}; this server serves {sorted(self.deciders)}, "
                                    "or omit model to let the server choose")
        return self.default_model

    def _run(self, call: Callable[[], Any]) -> tuple[Any, float]:
        start = time.perf_counter()
        try:
            out = call()
        except RequestError:
            raise
        except ValueError as e:
            raise RequestError(422, str(e)) from None
        except Exception:
            log.exception("inference failed")
            raise RequestError(500, "inference failed") from None
        return out, (time.perf_counter() - start) * 1e3

    def _finish(self, result: Mapping[str, Any]) -> dict[str, Any]:
        return strict_view(result) if self.jev_strict else with_confidence(result)


def _parse(raw: bytes) -> Any:
    if len(raw) > MAX_BODY_BYTES:
        raise RequestError(413, "request body too large")
    try:
        return json.loads(raw)
    except (ValueError, RecursionError):
        raise RequestError(400, "request body must be valid JSON") from None


def _refuse(body: Mapping[str, Any], unsupported: tuple[str, ...]) -> None:
    hooks = [k for k in HOOK_FIELDS if k in body]
    if hooks:
        raise RequestError(422, f"{', '.join(hooks)} cannot be set from a request; hooks belong to the server")
    sent = [k for k in unsupported if body.get(k) is not None]
    if sent:
        raise RequestError(422, f"{', '.join(sent)} is not supported by deciax")


def _token_cap(decider: Any) -> int:
    model = getattr(decider, "model", None)
    return int(getattr(model, "max_token_budget", 16384))


def _budgets(body: Mapping[str, Any], cap: int) -> dict[str, int]:
    out = {}
    for key in ("max_len", "head_max_len"):
        value = body.get(key)
        if value is None:
            continue
        if isinstance(value, bool) or not isinstance(value, int):
            raise RequestError(422, f"{key} must be an integer")
        if value <= 0:
            raise RequestError(422, f"{key} must be a positive integer")
        if value > cap:
            raise RequestError(422, f"{key} exceeds the server cap ({value} > {cap})")
        out[key] = value
    return out


def _timing(ms: float) -> dict[str, str]:
    return {"Server-Timing": f"inference;dur={ms:.2f}", "X-Inference-Time-Ms": f"{ms:.2f}"}


class _Handler(BaseHTTPRequestHandler):
    protocol_version = "HTTP/1.1"
    disable_nagle_algorithm = True

    def _send(self, response: Response) -> None:
        data = json.dumps(response.payload, ensure_ascii=False).encode("utf-8")
        self.send_response(response.status)
        self.send_header("Content-Type", "application/json")
        self.send_header("Content-Length", str(len(data)))
        for key, value in response.headers.items():
            self.send_header(key, value)
        self.end_headers()
        self.wfile.write(data)

    def _dispatch(self) -> None:
        body = b""
        if self.command == "POST":
            length = self.headers.get("Content-Length")
            if length is None:
                self.close_connection = True
                return self._send(_error(411, "Content-Length required"))
            try:
                n = int(length)
            except ValueError:
                self.close_connection = True
                return self._send(_error(400, "invalid Content-Length"))
            if n > MAX_BODY_BYTES:
                self.close_connection = True
                return self._send(_error(413, "request body too large"))
            body = self.rfile.read(n)
        headers = {k.lower(): v for k, v in self.headers.items()}
        self._send(self.server.service.handle(self.command, self.path, headers, body))  # type: ignore[attr-defined]

    do_GET = do_POST = do_PUT = do_DELETE = do_PATCH = _dispatch

    def log_message(self, format: str, *args: Any) -> None:  # noqa: A002
        log.info("%s - %s", self.address_string(), format % args)


class _Server(ThreadingHTTPServer):
    daemon_threads = True

    def __init__(self, address: tuple[str, int], service: Service) -> None:
        super().__init__(address, _Handler)
        self.service = service


def make_server(service: Service, host: str = "127.0.0.1", port: int = 8000) -> ThreadingHTTPServer:
    """A bound server, not yet serving (port 0 picks a free port)."""
    return _Server((host, port), service)


WARMUP_STATE = "warmup"
WARMUP_QUESTIONS = {"q": {"type": "noul", "instructions": "Is this a warmup request?"}}


def load_deciders(models: tuple[str, ...], *, dtype: str = "auto", impl: str = "auto",
                  seed: int = 0, warmup: bool = True) -> dict[str, Any]:
    """Load each model (a registered shape or a checkpoint directory) on the GPU, keyed by its name
    (a directory by its last path component)."""
    from deciax_amd.decider import load

    out: dict[str, Any] = {}
    for name in models:
        log.info("loading %s", name)
        key = Path(name).name if Path(name).is_dir() else name
        out[key] = load(name, dtype=dtype, impl=impl, seed=seed)  # type: ignore[arg-type]
        if warmup:
            out[key].decide(WARMUP_STATE, WARMUP_QUESTIONS)
    return out


def serve(host: str = "127.0.0.1", port: int = 8000, models: tuple[str, ...] = ("gemma2-9b",), *,
          default_model: str | None = None, api_key: str | None = None, max_concurrent: int = 16,
          jev_strict: bool = False, warmup: bool = True, dtype: str = "auto", impl: str = "auto",
          seed: int = 0) -> None:
    """Load the models and serve until interrupted (src/deciax/serve/app.py:391-423)."""
    deciders = load_deciders(models, dtype=dtype, impl=impl, seed=seed, warmup=warmup)
    from deciax_amd.backend import hip_device_arch

    first = next(iter(deciders))
    service = Service(deciders, default_model or first, api_key=api_key, max_concurrent=max_concurrent,
                      jev_strict=jev_strict, device=hip_device_arch() or "unknown")
    server = make_server(service, host, port)
    log.info("serving %s on http://%s:%d", sorted(deciders), *server.server_address[:2])
    try:
        server.serve_forever()
    finally:
        server.server_close()
