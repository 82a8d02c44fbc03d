'use strict';
// Gemma-3 chat template of the JavaScript host, same text as the reference's
// conversation.ts:6-52: an optional developer turn declaring the tools (only
// for a non-empty JSON array), then one <start_of_turn>role ... <end_of_turn>
// block per turn, then the opening of the model turn.

const ESC = '<escape>';

function declareTool(tool) {
  let d = '<start_function_declaration>declaration:' + tool.name + '{';
  d += 'description:' + ESC + tool.description + ESC;
  if (tool.parameters) {
    const props = Object.entries(tool.parameters.properties || {});
    d += ',parameters:{properties:{';
    d += props.map(function (kv) {
      const v = kv[1];
      let p = kv[0] + ':{description:' + ESC + v.description + ESC + ',type:' + ESC + v.type + ESC;
      if (v.enum) p += ',enum:[' + v.enum.map((e) => ESC + e + ESC).join(',') + ']';
      return p + '}';
    }).join(',');
    d += '}';
    if (tool.parameters.required) {
      d += ',required:[' + tool.parameters.required.map((r) => ESC + r + ESC).join(',') + ']';
    }
    d += ',type:' + ESC + tool.parameters.type + ESC + '}';
  }
  return d + '}<end_function_declaration>';
}

function buildChatPrompt(history, toolsJson) {
  let tools = null;
  if (toolsJson) {
    try {
      const parsed = JSON.parse(toolsJson);
      if (Array.isArray(parsed) && parsed.length > 0) tools = parsed;
    } catch (e) {
      tools = null;
    }
  }
  let prompt = '';
  if (tools) {
    prompt += '<start_of_turn>developer\nYou are a model that can do function calling with the following functions\n' +
      tools.map(declareTool).join('') + '\n<end_of_turn>\n';
  }
  for (const turn of history) prompt += '<start_of_turn>' + turn.role + '\n' + turn.text + '<end_of_turn>\n';
  return prompt + '<start_of_turn>model\n';
}

// Tokens that continue a conversation whose KV cache already holds the
// earlier turns (engine.ts:972-975): close the model turn, add the user turn,
// open the next model turn.
function turnSuffix(userText) {
  return '<end_of_turn>\n<start_of_turn>user\n' + userText + '<end_of_turn>\n<start_of_turn>model\n';
}

module.exports = { buildChatPrompt: buildChatPrompt, turnSuffix: turnSuffix };
