"""FastAPI routes of the front end (counterpart of litelang/apis/api_server.py).

Same routes and request body as the reference: `POST /generate` answers
{"result": [text, ...]} once the request has finished, `POST
/generate_stream` streams one `{"generated_text": text}` JSON object per
generated piece, each followed by a blank line (text/event-stream). The
reference's /generate reads `request.get()`, which its pydantic model does
not have; here it returns the generated pieces. A request the waiting room
refuses answers 503.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from typing import Iterator, Optional

from fastapi import FastAPI, HTTPException
from fastapi.responses import Response, StreamingResponse
from pydantic import BaseModel

from .http_server_manager import HttpServerManager, RequestRefused


@dataclass
class GObjs:
    http_server_manager: Optional[HttpServerManager] = None
    app: Optional[FastAPI] = None

    default_temperature = 1.0
    default_top_p = 1.0
    default_top_k = 1
    default_do_sample = False


app = FastAPI()
g_objs = GObjs(app=app)


class GenerateRequest(BaseModel):
    top_p: float = g_objs.default_top_p
    temperature: float = g_objs.default_temperature
    top_k: int = g_objs.default_top_k
    do_sample: bool = g_objs.default_do_sample
    prompt: str


def _manager() -> HttpServerManager:
    m = g_objs.http_server_manager
    if m is None:
        raise HTTPException(status_code=503, detail="no model is being served")
    return m


def _start(request: GenerateRequest) -> Iterator[str]:
    """The request's text generator, with its first step taken so that a
    refusal becomes an HTTP error before any byte is sent."""
    m = _manager()
    try:
        req = m.submit(request.prompt, request.top_p, request.top_k, request.temperature,
                       request.do_sample)
    except RequestRefused as e:
        raise HTTPException(status_code=503, detail=str(e))

    return m.stream(req)


@app.post("/generate")
def generate(request: GenerateRequest):
    output_prompts = list(_start(request))
    return Response(content=json.dumps({"result": output_prompts},
                                       ensure_ascii=False).encode("utf-8"),
                    media_type="application/json")


@app.post("/generate_stream")
def generate_stream(request: GenerateRequest):
    gen = _start(request)

    def stream_results():
        for text in gen:
            yield (json.dumps({"generated_text": text}, ensure_ascii=False) + "\n\n").encode("utf-8")

    return StreamingResponse(stream_results(), media_type="text/event-stream")


def serve(manager: HttpServerManager, host: str = "127.0.0.1", port: int = 8080) -> None:
    """Serve `app` for `manager` with uvicorn (blocks until the server stops)."""
    import uvicorn
    g_objs.http_server_manager = manager
    try:
        uvicorn.run(app, host=host, port=port)
    finally:
        manager.stop()
