"""FastAPI routes of the front end (counterpart of litelang/apis/api_server.py).

Same routes and request body fields as the reference: `POST /generate`
answers {"result": [text, ...]} once the request has finished, `POST
/generate_stream` streams one `{"generated_text": text}` JSON object per
generated piece, each followed by a blank line (text/event-stream). The
reference's /generate reads `request.get()`, which its pydantic model does
not have; here it returns the generated pieces. A request the waiting room
refuses answers 503, and so does any request while no model is attached.

The manager that serves the routes is attached with `attach(manager)` (or
`serve`, which attaches it and runs uvicorn) and detached with
`attach(None)`.
"""
from __future__ import annotations

import json
from typing import Iterator, Optional

from fastapi import FastAPI, HTTPException
from fastapi.responses import Response, StreamingResponse
from pydantic import BaseModel

from .http_server_manager import HttpServerManager, RequestRefused

# sampling defaults of a request body that leaves a field out (greedy
# decoding needs none of them; the scheduler records them per request)
SAMPLING_DEFAULTS = {"temperature": 1.0, "top_p": 1.0, "top_k": 1, "do_sample": False}

app = FastAPI()
_manager_ref: list[Optional[HttpServerManager]] = [None]


def attach(manager: Optional[HttpServerManager]) -> None:
    """Serve the routes from `manager` (None: answer 503 until one is attached)."""
    _manager_ref[0] = manager


def attached() -> Optional[HttpServerManager]:
    return _manager_ref[0]


class GenerateRequest(BaseModel):
    """JSON body of both routes (field names as the reference's)."""
    prompt: str
    temperature: float = SAMPLING_DEFAULTS["temperature"]
    top_p: float = SAMPLING_DEFAULTS["top_p"]
    top_k: int = SAMPLING_DEFAULTS["top_k"]
    do_sample: bool = SAMPLING_DEFAULTS["do_sample"]


def _pieces(body: GenerateRequest) -> Iterator[str]:
    """Submit the request and return its generator of text pieces. Submission
    happens here, before any response byte is sent, so that a refusal (or a
    missing model) becomes an HTTP 503."""
    manager = attached()
    if manager is None:
        raise HTTPException(status_code=503, detail="no model is being served")
    try:
        req = manager.submit(body.prompt, body.top_p, body.top_k, body.temperature,
                             body.do_sample)
    except RequestRefused as e:
        raise HTTPException(status_code=503, detail=str(e))
    return manager.stream(req)


def _json_bytes(obj) -> bytes:
    return json.dumps(obj, ensure_ascii=False).encode("utf-8")


@app.post("/generate")
def generate(body: GenerateRequest):
    return Response(content=_json_bytes({"result": list(_pieces(body))}),
                    media_type="application/json")


@app.post("/generate_stream")
def generate_stream(body: GenerateRequest):
    pieces = _pieces(body)
    events = (_json_bytes({"generated_text": text}) + b"\n\n" for text in pieces)
    return StreamingResponse(events, media_type="text/event-stream")


def serve(manager: HttpServerManager, host: str = "127.0.0.1", port: int = 8080) -> None:
    """Serve `app` for `manager` with uvicorn (blocks until the server stops)."""
    import uvicorn
    attach(manager)
    try:
        uvicorn.run(app, host=host, port=port)
    finally:
        attach(None)
        manager.stop()
